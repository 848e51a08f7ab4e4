"""IR tensors, the ``Operations`` builder and scalar operands.

Restates the assertions of the reference's tests/test_builder.py,
tests/test_tensor_metadata.py and tests/test_scalar_operands.py against this
package (imported through the reference's module names)."""

import numpy as np
import pytest

from orchestrator import (
    BroadcastSpec,
    ElementwiseOp,
    Layout,
    MatmulOp,
    Operations,
    ReductionOp,
    Scalar,
    Tensor,
    build_dag,
)


def _mlp_like():
    ops = Operations()
    ops.input("a", shape=(8, 16))
    ops.input("b", shape=(16, 4))
    ops.input("bias", shape=(1, 4))
    ops.matmul(a="a", b="b", out="c")
    ops.elementwise("add", out="d", operands=("c", "bias"), y_broadcast="row")
    ops.elementwise("exp", out="e", operands=("d",))
    ops.reduction("sum", out="r", x="e")
    return ops


# -- tensor metadata (reference tests/test_tensor_metadata.py) ---------------


def test_dense_strides_by_layout_and_rank():
    t = Tensor("a", (8, 16))
    assert t.layout is Layout.ROW_MAJOR and (t.row_stride, t.col_stride) == (16, 1)
    t = Tensor("a", (8, 16), layout=Layout.COL_MAJOR)
    assert (t.row_stride, t.col_stride) == (1, 8)
    t = Tensor("v", (8,))
    assert (t.row_stride, t.col_stride) == (1, 0)


def test_non_positive_dims_rejected():
    for shape in ((0, 4), (-1, 4)):
        with pytest.raises(ValueError, match="positive"):
            Tensor("z", shape)


def test_explicit_strides_kept():
    t = Tensor("a", (4, 4), row_stride=8, col_stride=1)
    assert (t.row_stride, t.col_stride) == (8, 1)


def test_transpose_swaps_metadata_and_shares_buffer():
    a = Tensor("a", (8, 16))
    at = a.transpose("a_T")
    assert (at.name, at.buffer_key, at.shape, at.layout) == ("a_T", "a", (16, 8), Layout.COL_MAJOR)
    assert (at.row_stride, at.col_stride) == (1, 16)
    back = at.transpose("a_TT")
    assert (back.shape, back.row_stride, back.col_stride, back.layout, back.buffer_key) == (
        a.shape, a.row_stride, a.col_stride, a.layout, "a"
    )


def test_transpose_needs_2d():
    with pytest.raises(ValueError, match="2D-only"):
        Tensor("v", (8,)).transpose("v_T")


def test_builder_input_layout():
    t = Operations().input("a", shape=(4, 4), layout=Layout.COL_MAJOR)
    assert t.layout is Layout.COL_MAJOR and (t.row_stride, t.col_stride) == (1, 4)


def test_broadcast_spec_parsing():
    with pytest.raises(ValueError):
        BroadcastSpec("rrow")
    assert BroadcastSpec.ROW == "row" and "row" == BroadcastSpec.ROW


# -- builder (reference tests/test_builder.py) -------------------------------


def test_matmul_output_shape_from_inputs():
    ops = Operations()
    ops.input("a", shape=(8, 16))
    ops.input("b", shape=(16, 4))
    c = ops.matmul(a="a", b="b", out="c")
    (op,) = ops.build()
    assert c.shape == (8, 4) and isinstance(op, MatmulOp) and op.out is c


def test_matmul_errors():
    with pytest.raises(ValueError, match="not declared"):
        Operations().matmul(a="x", b="y", out="z")
    ops = Operations()
    ops.input("a", shape=(4, 8))
    ops.input("b", shape=(7, 4))
    with pytest.raises(ValueError, match="contraction-axis"):
        ops.matmul(a="a", b="b", out="c")


def test_elementwise_shapes_and_broadcast_checks():
    ops = Operations()
    ops.input("x", shape=(4, 4))
    y = ops.elementwise("exp", out="y", operands=("x",))
    assert y.shape == (4, 4) and ops.build()[0].op == "exp"
    ops = Operations()
    ops.input("a", shape=(4, 8))
    ops.input("bias", shape=(1, 8))
    ops.elementwise("add", out="b", operands=("a", "bias"), y_broadcast="row")
    assert ops.tensors["b"].shape == (4, 8)
    ops = Operations()
    ops.input("a", shape=(4, 8))
    ops.input("bias", shape=(4, 1))
    with pytest.raises(ValueError, match="incompatible with y_broadcast"):
        ops.elementwise("add", out="b", operands=("a", "bias"), y_broadcast="row")


def test_elementwise_op_and_arity_errors():
    ops = Operations()
    ops.input("x", shape=(2, 2))
    with pytest.raises(ValueError):
        ops.elementwise("nope", out="y", operands=("x",))
    with pytest.raises(ValueError, match="arity"):
        ops.elementwise("exp", out="y", operands=("x", "x"))


def test_reduction_last_axis_only():
    ops = Operations()
    ops.input("x", shape=(8, 16))
    r = ops.reduction("sum", out="r", x="x")
    assert r.shape == (8,) and isinstance(ops.build()[0], ReductionOp)
    with pytest.raises(ValueError, match="last axis"):
        ops.reduction("sum", out="r2", x="x", axis=0)


def test_ssa_and_declaration_errors():
    ops = Operations()
    ops.input("x", shape=(4, 4))
    ops.elementwise("exp", out="y", operands=("x",))
    with pytest.raises(ValueError, match="SSA"):
        ops.elementwise("log", out="y", operands=("x",))
    with pytest.raises(ValueError, match="not declared"):
        Operations().elementwise("exp", out="y", operands=("ghost",))


def test_from_numpy_storage_and_dtype_checks():
    ops = Operations()
    ops.input("A", shape=(4, 4), row_stride=8, col_stride=1)
    with pytest.raises(ValueError, match="can address"):
        ops.from_numpy(np.zeros((4, 4), dtype=np.float32), "A")
    with pytest.raises(ValueError, match="float32"):
        Operations().from_numpy(np.zeros((4, 4), dtype=np.float64), "A")
    ops = Operations()
    ops.from_numpy(np.zeros((4, 4), dtype=np.float32), "A")
    ops.transpose("A", out="At")
    with pytest.raises(ValueError, match="view"):
        ops.from_numpy(np.zeros((4, 4), dtype=np.float32), "At")


def test_program_roundtrip():
    ops = _mlp_like()
    assert [type(op).__name__ for op in ops.build()] == [
        "MatmulOp", "ElementwiseOp", "ElementwiseOp", "ReductionOp"
    ]
    assert ops.tensors["r"].shape == (8,)


# -- scalar operands (reference tests/test_scalar_operands.py) ---------------


def test_relu_scalar_operand():
    ops = Operations()
    ops.input("x", shape=(4, 4))
    ops.elementwise("max", out="y", operands=("x", 0.0))
    (op,) = ops.build()
    assert isinstance(op, ElementwiseOp) and op.op == "max"
    assert isinstance(op.operands[1], Scalar) and op.operands[1].value == 0.0
    assert op.inputs == (op.operands[0],)
    dag = build_dag(ops.build())
    assert dag.inputs == frozenset({"x"}) and dag.outputs == frozenset({"y"})


def test_scalar_operand_rules():
    ops = Operations()
    ops.input("x", shape=(4, 4))
    with pytest.raises(ValueError, match="cannot be set for a Scalar"):
        ops.elementwise("max", out="y", operands=("x", 0.0), y_broadcast=BroadcastSpec.SCALAR)
    with pytest.raises(ValueError, match=r"operand\[0\] must be a tensor"):
        ops.elementwise("max", out="y", operands=(0.0, "x"))
    with pytest.raises(ValueError, match="must be a tensor name"):
        ops.elementwise("max", out="y", operands=("x", [1.0]))
    with pytest.raises(ValueError, match="must be a tensor name"):
        ops.elementwise("max", out="y", operands=("x", True))


def test_string_broadcast_is_enum():
    ops = Operations()
    ops.input("a", shape=(4, 8))
    ops.input("bias", shape=(1, 8))
    ops.elementwise("add", out="b", operands=("a", "bias"), y_broadcast="row")
    assert ops.build()[0].y_broadcast is BroadcastSpec.ROW


# -- DAG (reference tests/test_dag.py) ---------------------------------------


def test_dag_maps_inputs_outputs():
    program = _mlp_like().build()
    dag = build_dag(program)
    assert set(dag.producer_of) == {"c", "d", "e", "r"}
    assert isinstance(dag.producer_of["c"], MatmulOp)
    assert isinstance(dag.producer_of["r"], ReductionOp)
    assert dag.consumers_of["c"] == (dag.producer_of["d"],)
    assert dag.consumers_of["e"] == (dag.producer_of["r"],)
    assert "r" not in dag.consumers_of
    assert dag.inputs == frozenset({"a", "b", "bias"}) and dag.outputs == frozenset({"r"})
    assert dag.unique_consumer("c") is dag.producer_of["d"]
    assert dag.topo_order() == program
    order = dag.topo_order()
    order.clear()
    assert dag.topo_order() == program


def test_dag_unique_consumer_none_cases():
    ops = Operations()
    ops.input("x", shape=(4, 4))
    ops.elementwise("exp", out="y", operands=("x",))
    ops.elementwise("log", out="z", operands=("x",))
    dag = build_dag(ops.build())
    assert dag.unique_consumer("x") is None and dag.unique_consumer("y") is None


def test_dag_ssa_and_order_violations():
    x, y, z = Tensor("x", (4, 4)), Tensor("y", (4, 4)), Tensor("z", (4, 4))
    with pytest.raises(ValueError, match="SSA violation"):
        build_dag([ElementwiseOp(out=y, op="exp", operands=(x,)), ElementwiseOp(out=y, op="log", operands=(x,))])
    with pytest.raises(ValueError, match="def-after-use"):
        build_dag([ElementwiseOp(out=z, op="exp", operands=(y,)), ElementwiseOp(out=y, op="log", operands=(x,))])
