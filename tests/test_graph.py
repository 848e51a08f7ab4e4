"""Vertex graph substrate: construction, replace, topo order, flatten and the
dependency check (assertions of the reference's tests/test_graph.py)."""

import pytest

from orchestrator import Operations
from orchestrator.graph import Graph, Vertex
from orchestrator.ir import MatmulOp


def _chain():
    ops = Operations()
    ops.input("a", shape=(8, 16))
    ops.input("b", shape=(16, 4))
    ops.input("bias", shape=(1, 4))
    ops.matmul(a="a", b="b", out="c")
    ops.elementwise("add", out="d", operands=("c", "bias"), y_broadcast="row")
    ops.elementwise("exp", out="e", operands=("d",))
    ops.reduction("sum", out="r", x="e")
    return ops.build()


def _named(g: Graph) -> dict:
    return {v.ops[0].out.name: v for v in g.vertices if v.is_primitive}


def test_one_primitive_vertex_per_op_with_boundaries():
    prog = _chain()
    g = Graph.from_program(prog)
    assert len(g.vertices) == len(prog) and all(v.is_primitive for v in g.vertices)
    v = _named(g)
    assert v["c"].inputs == ("a", "b") and v["c"].outputs == ("c",)
    assert set(v["d"].inputs) == {"c", "bias"} and v["d"].outputs == ("d",)
    assert v["e"].inputs == ("d",) and v["r"].outputs == ("r",)
    assert g.program_outputs == frozenset({"r"})


def test_program_outputs_override_and_dead_outputs():
    prog = _chain()
    g = Graph.from_program(prog, program_outputs=frozenset({"d", "r"}))
    assert g.program_outputs == frozenset({"d", "r"})
    g = Graph.from_program(prog, program_outputs=frozenset())
    v = _named(g)
    assert v["r"].outputs == () and v["c"].outputs == ("c",)


def test_view_is_an_external_input():
    ops = Operations()
    ops.input("X", shape=(4, 8))
    ops.input("Ybase", shape=(8, 4))
    ops.transpose("Ybase", out="Yview")
    ops.elementwise("add", out="Z", operands=("X", "Yview"))
    g = Graph.from_program(ops.build())
    (z,) = g.vertices
    assert set(z.inputs) == {"X", "Yview"} and z.outputs == ("Z",)


def test_vertex_identity_helpers():
    g = Graph.from_program(_chain())
    for v in g.vertices:
        assert v.op_ids == frozenset(id(op) for op in v.ops)
    v = _named(g)
    after = g.replace(absorbed=(v["d"], v["e"]), ops=(v["d"].ops[0], v["e"].ops[0]))
    assert not next(x for x in after.vertices if len(x.ops) == 2).is_primitive


def test_replace_boundaries():
    prog = _chain()
    g = Graph.from_program(prog)
    v = _named(g)
    after = g.replace(absorbed=(v["d"], v["e"]), ops=(v["d"].ops[0], v["e"].ops[0]))
    assert len(after.vertices) == len(g.vertices) - 1
    sv = next(x for x in after.vertices if len(x.ops) == 2)
    assert set(sv.inputs) == {"c", "bias"} and sv.outputs == ("e",)
    everything = g.replace(absorbed=g.vertices, ops=tuple(prog))
    (only,) = everything.vertices
    assert set(only.inputs) == {"a", "b", "bias"} and only.outputs == ("r",)
    cd = g.replace(absorbed=(v["c"], v["d"]), ops=(v["c"].ops[0], v["d"].ops[0]))
    sv = next(x for x in cd.vertices if len(x.ops) == 2)
    assert set(sv.inputs) == {"a", "b", "bias"} and sv.outputs == ("d",)


def test_replace_keeps_program_output_visible():
    g = Graph.from_program(_chain(), program_outputs=frozenset({"d", "r"}))
    v = _named(g)
    after = g.replace(absorbed=(v["d"], v["e"]), ops=(v["d"].ops[0], v["e"].ops[0]))
    sv = next(x for x in after.vertices if len(x.ops) == 2)
    assert set(sv.outputs) == {"d", "e"}


def test_replace_precondition_errors():
    g = Graph.from_program(_chain())
    other = Graph.from_program(_chain())
    v0 = g.vertices[0]
    with pytest.raises(ValueError, match="empty"):
        g.replace(absorbed=(), ops=())
    with pytest.raises(ValueError, match="not in this graph"):
        g.replace(absorbed=(other.vertices[0],), ops=other.vertices[0].ops)
    with pytest.raises(ValueError, match="duplicate"):
        g.replace(absorbed=(v0, v0), ops=v0.ops)
    with pytest.raises(ValueError, match="ops does not match"):
        g.replace(absorbed=(v0,), ops=())
    v = _named(g)
    with pytest.raises(ValueError, match="program order"):
        g.replace(absorbed=(v["d"], v["e"]), ops=(v["e"].ops[0], v["d"].ops[0]))
    with pytest.raises(ValueError, match="cycle|convex"):
        g.replace(absorbed=(v["c"], v["r"]), ops=(v["c"].ops[0], v["r"].ops[0]))


def test_replace_is_functional():
    g = Graph.from_program(_chain())
    before = g.vertices
    v = _named(g)
    g.replace(absorbed=(v["d"], v["e"]), ops=(v["d"].ops[0], v["e"].ops[0]))
    assert g.vertices is before


def test_topo_sort_and_flatten():
    prog = _chain()
    g = Graph.from_program(prog)
    assert [v.ops[0] for v in g.topo_sort()] == list(prog)
    assert g.flatten() == tuple(prog)
    ops = Operations()
    ops.input("X", shape=(4, 4))
    ops.elementwise("exp", out="A", operands=("X",))
    ops.elementwise("log", out="B", operands=("X",))
    g2 = Graph.from_program(ops.build())
    order = g2.topo_sort()
    assert order == g2.topo_sort()
    assert [v.ops[0].out.name for v in order] == ["A", "B"]
    assert tuple(v.ops[0].out.name for v in g2.consumers_of("X")) == ("A", "B")
    assert g2.consumers_of("nope") == ()


def test_topo_sort_detects_cycle():
    ops = Operations()
    ops.input("X", shape=(4, 4))
    ops.elementwise("exp", out="Y", operands=("X",))
    ops.elementwise("log", out="Z", operands=("Y",))
    p = ops.build()
    g = Graph(
        vertices=(Vertex(ops=(p[0],), inputs=("Z",), outputs=("Y",)), Vertex(ops=(p[1],), inputs=("Y",), outputs=("Z",))),
        op_index={id(op): i for i, op in enumerate(p)},
        program_outputs=frozenset({"Z"}),
    )
    with pytest.raises(ValueError, match="cycle"):
        g.topo_sort()


def test_dependency_check():
    prog = _chain()
    g = Graph.from_program(prog)
    g.check_dependencies(prog)
    assert g.preserves_dependencies(prog)
    v = _named(g)
    g.replace(absorbed=(v["d"], v["e"]), ops=(v["d"].ops[0], v["e"].ops[0])).check_dependencies(prog)
    truncated = Graph(vertices=g.vertices[:-1], op_index=g.op_index, program_outputs=g.program_outputs)
    with pytest.raises(ValueError, match="missing"):
        truncated.check_dependencies(prog)
    mm, add, exp, red = prog
    bad = Graph(
        vertices=(
            Vertex(ops=(add, mm), inputs=("a", "b", "bias"), outputs=("d",)),
            Vertex(ops=(exp,), inputs=("d",), outputs=("e",)),
            Vertex(ops=(red,), inputs=("e",), outputs=("r",)),
        ),
        op_index={id(op): i for i, op in enumerate(prog)},
        program_outputs=frozenset({"r"}),
    )
    with pytest.raises(ValueError, match="dependency violated"):
        bad.check_dependencies(prog)
    assert not bad.preserves_dependencies(prog)


def test_producer_lookup():
    g = Graph.from_program(_chain())
    p = g.producer_of("c")
    assert p is not None and isinstance(p.ops[0], MatmulOp)
    assert g.producer_of("a") is None and g.producer_of("nope") is None


def test_absorb_into_and_remove_vertex():
    ops = Operations()
    ops.input("X", shape=(8, 8))
    ops.input("B1", shape=(8, 8))
    ops.input("B2", shape=(8, 8))
    ops.elementwise("max", out="Xr", operands=("X", 0.0))
    ops.matmul(a="Xr", b="B1", out="C1")
    ops.matmul(a="Xr", b="B2", out="C2")
    prog = ops.build()
    g = Graph.from_program(prog)
    relu, m1, m2 = g.vertices
    g1 = g.absorb_into(m1, relu.ops)
    grown = next(v for v in g1.vertices if m1.ops[0] in v.ops)
    assert grown.ops == (prog[0], prog[1]) and set(grown.inputs) == {"X", "B1"}
    with pytest.raises(ValueError, match="still consumed"):
        g1.remove_vertex(relu)
    g2 = g1.absorb_into(m2, relu.ops)
    g3 = g2.remove_vertex(relu)
    assert len(g3.vertices) == 2
    g3.check_dependencies(prog)
    with pytest.raises(ValueError, match="empty"):
        g.absorb_into(m1, ())
