"""Classify a fused vertex into a ``FusionStrategy`` and split its ops into
the pieces the templates consume (reference:
src/orchestrator/assembly/decision.py:52-224).  Pure function of
``vertex.ops``; the labels are the reference's."""

from __future__ import annotations

from dataclasses import dataclass

from metellus_amd.compute.elementwise.elementwise import TERNARY_EXPRESSIONS
from metellus_amd.orchestrator.graph import Vertex
from metellus_amd.orchestrator.ir import ElementwiseOp, MatmulOp, Op, ReductionOp, Scalar, ShapeOp, Tensor
from metellus_amd.orchestrator.kernel_group import FusionStrategy


@dataclass
class DecisionView:
    strategy: FusionStrategy
    anchor: MatmulOp | ReductionOp | None = None
    prologue_a: tuple[ElementwiseOp, ...] = ()
    prologue_b: tuple[ElementwiseOp, ...] = ()
    epilogue: tuple[ElementwiseOp, ...] = ()
    chain_only: tuple[ElementwiseOp, ...] = ()
    shape_op: ShapeOp | None = None
    ops: tuple[Op, ...] = ()
    anchors: tuple[MatmulOp, ...] = ()
    merge_elem: ElementwiseOp | None = None
    # the merge ops in program order (the reference's one op, or a chain from
    # the MULTI_ANCHOR_MERGE_CHAINS extension); merge_elem is the last
    merge_chain: tuple[ElementwiseOp, ...] = ()
    shared_a: bool = False
    prologues_a: tuple[tuple[ElementwiseOp, ...], ...] = ()
    prologues_b: tuple[tuple[ElementwiseOp, ...], ...] = ()
    # MATMUL_REDUCTION_EPILOGUE: the last-axis reduction of the matmul's
    # (epilogue) output computed in the same kernel
    reduction: ReductionOp | None = None


def trace_prologue(target_name: str, candidates: tuple[Op, ...]) -> tuple[ElementwiseOp, ...]:
    """Walk back from ``target_name`` through elementwise producers in
    ``candidates`` along primary operands; returns the chain head-first."""
    made = {op.out.name: op for op in candidates}
    chain: list[ElementwiseOp] = []
    cur = target_name
    while True:
        prod = made.get(cur)
        if not isinstance(prod, ElementwiseOp):
            break
        chain.append(prod)
        head = prod.operands[0]
        if not isinstance(head, Tensor):
            break
        cur = head.name
    chain.reverse()
    return tuple(chain)


def is_lane_agnostic_pred(op: ElementwiseOp) -> bool:
    """No tensor secondary operands (and not ternary)."""
    if op.op in TERNARY_EXPRESSIONS:
        return False
    return all(isinstance(o, Scalar) for o in op.operands[1:])


def _classify_multi_anchor(ops: tuple[Op, ...], anchors: tuple[MatmulOp, ...]) -> DecisionView:
    assert len(anchors) == 2 and not any(isinstance(op, ReductionOp) for op in ops), (
        "v0: multi-anchor vertex must have exactly 2 matmul anchors and no reduction anchors"
    )
    a0, a1 = anchors
    i0, i1 = ops.index(a0), ops.index(a1)
    tail = ops[max(i0, i1) + 1 :]
    if len(tail) > 1:
        from metellus_amd.orchestrator import fusion

        assert fusion.MULTI_ANCHOR_MERGE_CHAINS and all(isinstance(op, ElementwiseOp) for op in tail), (
            "v0: multi-anchor vertex has exactly one merge elem"
        )
    assert tail and isinstance(tail[0], ElementwiseOp), "v0: multi-anchor vertex has exactly one merge elem"
    merge = tail[-1]
    pre0 = tuple(op for op in ops[:i0] if isinstance(op, ElementwiseOp))
    pre1 = tuple(op for op in ops[:i1] if isinstance(op, ElementwiseOp))
    pro_a = (trace_prologue(a0.a.name, pre0), trace_prologue(a1.a.name, pre1))
    pro_b = (trace_prologue(a0.b.name, pre0), trace_prologue(a1.b.name, pre1))
    covered = {id(op) for chain in (*pro_a, *pro_b) for op in chain}
    covered |= {id(op) for op in tail}
    for op in ops:
        if isinstance(op, ElementwiseOp):
            assert id(op) in covered, (
                f"v0: pre-anchor elementwise op {op.out.name!r} not absorbed by any anchor prologue"
            )
    # Shared A only without A prologues (the reference compares names).
    shared = a0.a.name == a1.a.name and a0.a.shape == a1.a.shape and not pro_a[0] and not pro_a[1]
    return DecisionView(
        strategy=FusionStrategy.DIAMOND_SHARED if shared else FusionStrategy.MULTI_PRODUCER_CONVERGENT,
        anchors=anchors,
        merge_elem=merge,
        merge_chain=tuple(tail),
        shared_a=shared,
        prologues_a=pro_a,
        prologues_b=pro_b,
        ops=ops,
    )


def classify(vertex: Vertex) -> DecisionView:
    ops = vertex.ops
    shape_op = next((op for op in ops if isinstance(op, ShapeOp)), None)
    if shape_op is not None:
        assert len(ops) == 1, "ShapeOp must be standalone (no fusion in v0)"
        return DecisionView(strategy=FusionStrategy.STANDALONE_SHAPE, shape_op=shape_op, ops=ops)

    matmuls = tuple(op for op in ops if isinstance(op, MatmulOp))
    if len(matmuls) >= 2:
        return _classify_multi_anchor(ops, matmuls)

    anchor = next((op for op in ops if isinstance(op, (MatmulOp, ReductionOp))), None)
    if anchor is None:
        assert all(isinstance(op, ElementwiseOp) for op in ops)
        chain = tuple(ops)
        strategy = FusionStrategy.ELEMENTWISE_CHAIN if len(chain) > 1 else FusionStrategy.STANDALONE_ELEMENTWISE
        return DecisionView(strategy=strategy, chain_only=chain, ops=ops)

    at = ops.index(anchor)
    pre, post = ops[:at], ops[at + 1 :]
    if isinstance(anchor, MatmulOp) and post and isinstance(post[-1], ReductionOp):
        return _classify_matmul_reduction(ops, anchor, pre, post)
    epilogue = tuple(op for op in post if isinstance(op, ElementwiseOp))
    if isinstance(anchor, MatmulOp):
        pro_a = trace_prologue(anchor.a.name, pre)
        pro_b = trace_prologue(anchor.b.name, pre)
        if epilogue and all(is_lane_agnostic_pred(e) for e in epilogue):
            strategy = FusionStrategy.MATMUL_EPILOGUE_REGISTER
        elif epilogue:
            strategy = FusionStrategy.MATMUL_EPILOGUE_TG
        elif pro_a or pro_b:
            strategy = FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL
        else:
            strategy = FusionStrategy.STANDALONE_MATMUL
        return DecisionView(
            strategy=strategy, anchor=anchor, prologue_a=pro_a, prologue_b=pro_b, epilogue=epilogue, ops=ops
        )
    pro = trace_prologue(anchor.input.name, pre)
    if pro:
        strategy = FusionStrategy.ELEMENTWISE_PROLOGUE_REDUCTION
    elif epilogue:
        strategy = FusionStrategy.REDUCTION_EPILOGUE
    else:
        strategy = FusionStrategy.STANDALONE_REDUCTION
    return DecisionView(strategy=strategy, anchor=anchor, prologue_a=pro, epilogue=epilogue, ops=ops)


def _classify_matmul_reduction(ops, anchor: MatmulOp, pre, post) -> DecisionView:
    """(Extension, ``fusion.MATMUL_REDUCTION_EPILOGUES``.)  A matmul, its
    lane-agnostic register epilogue and a last-axis reduction of the
    epilogue's output, in one kernel that writes both."""
    from metellus_amd.orchestrator import fusion

    red = post[-1]
    epilogue = post[:-1]
    out = epilogue[-1].out if epilogue else anchor.out
    assert fusion.MATMUL_REDUCTION_EPILOGUES, "v0: a matmul vertex holds no reduction"
    assert not pre and all(isinstance(op, ElementwiseOp) and is_lane_agnostic_pred(op) for op in epilogue), (
        "matmul -> reduction epilogue: no prologue, lane-agnostic epilogue only"
    )
    assert red.input.name == out.name, "matmul -> reduction epilogue: the reduction reads the matmul's output"
    return DecisionView(
        strategy=FusionStrategy.MATMUL_REDUCTION_EPILOGUE,
        anchor=anchor,
        epilogue=tuple(epilogue),
        reduction=red,
        ops=ops,
    )
