"""Fusion: Program -> topo-ordered tuple of ``Vertex``es, one kernel each.

The rules, their priority and the budget gate are the reference's
(src/orchestrator/fusion.py:1-545); only the LDS cap differs (163,840 B on
gfx950, see ``aliasing.TGMEM_CAP_BYTES``).

Passes, highest priority first; after every rewrite the driver restarts at
the top, until nothing fires ("saturation"):

1. ``try_elem_chain_fuse``        elem -> elem (unique consumer, primary edge)
2. ``try_multi_producer_fuse``    matmul, matmul -> binary merge elem
3. ``try_epilogue_absorb``        matmul/reduction -> elem (unique consumer)
4. ``try_prologue_absorb_single`` elem -> anchor input (unique consumer)
5. ``try_prologue_absorb_multi``  lane-agnostic elem recomputed in 2+ anchors

Two extensions beyond the reference, off by default:

* ``MULTI_ANCHOR_MERGE_CHAINS``: ``try_multi_producer_chain_fuse`` runs
  between 1 and 2 and merges two matmuls through a chain of elementwise ops
  instead of one (the MLP gate ``silu(X @ W1) * (X @ W2)``);
* ``MATMUL_REDUCTION_EPILOGUES``: once the passes above are saturated,
  ``try_matmul_reduction_fuse`` (the only late pass) joins a last-axis
  reduction to the matmul vertex producing its input (attention's
  ``max(Q @ K^T * s)``), so the reference's passes never see that vertex.

Budget gate: each rewrite's new vertices are assembled and their LDS plan
measured; a rewrite that exceeds the cap is blacklisted by its op-id
signature and fusion restarts from the primitive graph.
"""

from __future__ import annotations

from metellus_amd.compute.elementwise.elementwise import (
    BINARY_EXPRESSIONS,
    TERNARY_EXPRESSIONS,
    UNARY_EXPRESSIONS,
    BroadcastSpec,
)
from metellus_amd.orchestrator.aliasing import (  # noqa: F401 (TGMEM_CAP_BYTES is patched by tests)
    TGMEM_CAP_BYTES,
    TgmemOverflowError,
    compute_group_budget,
)
from metellus_amd.orchestrator.graph import Graph, Vertex
from metellus_amd.orchestrator.ir import (
    ElementwiseOp,
    MatmulOp,
    Op,
    Program,
    ReductionOp,
    Scalar,
    Tensor,
)

Blacklist = frozenset  # frozenset[frozenset[int]] of op-id signatures


# ---------------------------------------------------------------------------
# Eligibility policies (reference: fusion.py:56-116)
# ---------------------------------------------------------------------------


def _is_unary(op: ElementwiseOp) -> bool:
    return op.op in UNARY_EXPRESSIONS


def _is_binary(op: ElementwiseOp) -> bool:
    return op.op in BINARY_EXPRESSIONS


def _is_ternary(op: ElementwiseOp) -> bool:
    return op.op in TERNARY_EXPRESSIONS


def _is_lane_agnostic(op: ElementwiseOp) -> bool:
    """Every secondary operand is a Scalar (or there is none): the value at
    a position depends only on the primary at that position."""
    return not _is_ternary(op) and all(isinstance(o, Scalar) for o in op.operands[1:])


def _epilogue_eligible_matmul(elem: ElementwiseOp, primary_name: str) -> bool:
    if _is_ternary(elem):
        return False
    head = elem.operands[0]
    return isinstance(head, Tensor) and head.name == primary_name


def _prologue_eligible(elem: ElementwiseOp) -> bool:
    return _is_unary(elem) or _is_binary(elem)


def _reduction_epilogue_eligible(elem: ElementwiseOp) -> bool:
    """Unary, or binary with a Scalar second operand (a 1-D reduction output
    has no broadcastable tensor partner)."""
    if _is_unary(elem):
        return True
    return _is_binary(elem) and isinstance(elem.operands[1], Scalar)


def _anchor_of(vertex: Vertex) -> Op | None:
    return next((op for op in vertex.ops if isinstance(op, (MatmulOp, ReductionOp))), None)


def _is_elementwise_vertex(vertex: Vertex) -> bool:
    return bool(vertex.ops) and all(isinstance(op, ElementwiseOp) for op in vertex.ops)


def _primary_name(elem: ElementwiseOp) -> str | None:
    head = elem.operands[0]
    return head.name if isinstance(head, Tensor) else None


def _sole_consumer(graph: Graph, name: str) -> Vertex | None:
    readers = graph.consumers_of(name)
    return readers[0] if len(readers) == 1 else None


def _by_position(graph: Graph, ops) -> tuple[Op, ...]:
    return tuple(sorted(ops, key=lambda op: graph.op_index[id(op)]))


def _anchor_boundary_input_names(anchor: Op, anchor_vertex: Vertex) -> set[str]:
    """Names whose producer could still be folded into ``anchor``'s input
    loads.  For a fresh anchor these are its operands; once a prologue chain
    is absorbed on an operand, the boundary moves back to that chain's
    head primary (reference: fusion.py:396-427)."""
    if isinstance(anchor, MatmulOp):
        starts = [anchor.a.name, anchor.b.name]
    elif isinstance(anchor, ReductionOp):
        starts = [anchor.input.name]
    else:
        return set()
    before = anchor_vertex.ops[: anchor_vertex.ops.index(anchor)]
    made_before = {op.out.name: op for op in before}
    boundary: set[str] = set()
    for name in starts:
        cur = name
        while True:
            prod = made_before.get(cur)
            if not isinstance(prod, ElementwiseOp):
                break
            nxt = _primary_name(prod)
            if nxt is None:
                break
            cur = nxt
        boundary.add(cur)
    return boundary


# ---------------------------------------------------------------------------
# Passes: each returns a rewritten graph for its first match, else None.
# ---------------------------------------------------------------------------


def try_elem_chain_fuse(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """U (elem) -> V (elem): U's last output is read only by V, as V's first
    op's primary; V's first op is not ternary."""
    for u in graph.vertices:
        if not _is_elementwise_vertex(u):
            continue
        tail = u.ops[-1].out.name
        if tail not in u.outputs:
            continue
        v = _sole_consumer(graph, tail)
        if v is None or not _is_elementwise_vertex(v):
            continue
        head = v.ops[0]
        if _is_ternary(head) or _primary_name(head) != tail:
            continue
        if (u.op_ids | v.op_ids) in blacklist:
            continue
        return graph.replace(absorbed=(u, v), ops=u.ops + v.ops)
    return None


def try_epilogue_absorb(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """A (matmul/reduction vertex) -> V (elem): V alone reads A's last
    output, through V's first op's primary."""
    for a in graph.vertices:
        anchor = _anchor_of(a)
        if anchor is None:
            continue
        tail = a.ops[-1].out.name
        if tail not in a.outputs:
            continue
        v = _sole_consumer(graph, tail)
        if v is None or not _is_elementwise_vertex(v):
            continue
        head = v.ops[0]
        if isinstance(anchor, MatmulOp):
            if not _epilogue_eligible_matmul(head, tail):
                continue
        elif not (_reduction_epilogue_eligible(head) and _primary_name(head) == tail):
            continue
        if (a.op_ids | v.op_ids) in blacklist:
            continue
        return graph.replace(absorbed=(a, v), ops=a.ops + v.ops)
    return None


def try_prologue_absorb_single(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """V (elem, unary/binary ops only) -> A: A alone reads V's last output,
    at one of A's anchors' load boundaries."""
    for v in graph.vertices:
        if not _is_elementwise_vertex(v):
            continue
        tail = v.ops[-1].out.name
        if tail not in v.outputs:
            continue
        a = _sole_consumer(graph, tail)
        if a is None:
            continue
        anchors = [op for op in a.ops if isinstance(op, (MatmulOp, ReductionOp))]
        if not anchors:
            continue
        boundary: set[str] = set()
        for anc in anchors:
            boundary |= _anchor_boundary_input_names(anc, a)
        if tail not in boundary:
            continue
        if not all(_prologue_eligible(op) for op in v.ops):
            continue
        if (v.op_ids | a.op_ids) in blacklist:
            continue
        return graph.replace(absorbed=(v, a), ops=_by_position(graph, (*v.ops, *a.ops)))
    return None


def try_multi_producer_fuse(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """Single binary elem merging the outputs of two distinct pure-matmul
    vertices of equal output shape, each read only by the merge
    (y_broadcast NONE, both operands tensors)."""
    for v in graph.vertices:
        if not _is_elementwise_vertex(v) or len(v.ops) != 1:
            continue
        merge = v.ops[0]
        if not _is_binary(merge) or merge.y_broadcast is not BroadcastSpec.NONE:
            continue
        x, y = merge.operands[0], merge.operands[1]
        if not (isinstance(x, Tensor) and isinstance(y, Tensor)):
            continue
        px, py = graph.producer_of(x.name), graph.producer_of(y.name)
        if px is None or py is None or px is py:
            continue
        if len(px.ops) != 1 or len(py.ops) != 1:
            continue
        mx, my = px.ops[0], py.ops[0]
        if not (isinstance(mx, MatmulOp) and isinstance(my, MatmulOp)):
            continue
        if len(graph.consumers_of(x.name)) != 1 or len(graph.consumers_of(y.name)) != 1:
            continue
        if mx.out.shape != my.out.shape:
            continue
        if (px.op_ids | py.op_ids | v.op_ids) in blacklist:
            continue
        ops = _by_position(graph, (*px.ops, *py.ops, *v.ops))
        return graph.replace(absorbed=(px, py, v), ops=ops)
    return None


# Extension beyond the reference's rules, off by default: the two matmuls
# of a multi-anchor kernel may merge through a chain of elementwise ops --
# each op reading the two matmul outputs, scalars and earlier ops of the
# chain, e.g. silu(X @ W1) * (X @ W2) = (h1 * recip(1 + exp(-h1))) * h2 --
# instead of one binary op.  The reference fuses only the one-op merge
# (fusion.py:219-247 here, its try_multi_producer_fuse); with this flag the
# MLP block's gate becomes one DIAMOND_SHARED kernel writing the gated
# product, and the matmul after it loads that product directly.
MULTI_ANCHOR_MERGE_CHAINS = False


def try_multi_producer_chain_fuse(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """(Extension, ``MULTI_ANCHOR_MERGE_CHAINS``.)  Two single-matmul vertices
    of equal output shape and the elementwise vertices that read them: the
    merge set grows from the matmuls' readers through the readers of its own
    values, stopping at the first reader that is not elementwise.  It fuses
    when every tensor it reads is one of the two matmul outputs or its own
    (no other tensors), it comes after both matmuls in program order, and
    exactly one of its values -- its last op's -- is read outside it or is a
    program output.  The one-op merge is left to the reference's pass."""
    if not MULTI_ANCHOR_MERGE_CHAINS:
        return None
    mats = [v for v in graph.vertices if len(v.ops) == 1 and isinstance(v.ops[0], MatmulOp)]
    for i, pa in enumerate(mats):
        for pb in mats[i + 1:]:
            ma, mb = pa.ops[0], pb.ops[0]
            if ma.out.shape != mb.out.shape:
                continue
            seeds = (ma.out.name, mb.out.name)
            members: list[Vertex] = []
            queue = [c for name in seeds for c in graph.consumers_of(name)]
            while queue:
                v = queue.pop()
                if any(v is m for m in members) or v is pa or v is pb or not _is_elementwise_vertex(v):
                    continue
                members.append(v)
                queue.extend(c for name in v.outputs for c in graph.consumers_of(name))
            if not members or (len(members) == 1 and len(members[0].ops) == 1):
                continue
            chain = _by_position(graph, tuple(op for v in members for op in v.ops))
            made = set(seeds) | {op.out.name for op in chain}
            if any(isinstance(o, Tensor) and o.name not in made for op in chain for o in op.operands):
                continue
            last_anchor = max(graph.op_index[id(ma)], graph.op_index[id(mb)])
            if graph.op_index[id(chain[0])] < last_anchor:
                continue
            inside = {id(v) for v in (pa, pb, *members)}
            escaping = {
                name for name in made
                if name in graph.program_outputs or any(id(c) not in inside for c in graph.consumers_of(name))
            }
            if escaping != {chain[-1].out.name}:
                continue
            ops = _by_position(graph, (ma, mb, *chain))
            if frozenset(id(op) for op in ops) in blacklist:
                continue
            return graph.replace(absorbed=(pa, pb, *members), ops=ops)
    return None


def _should_recompute(elem: ElementwiseOp) -> bool:
    """Recompute a shared prologue only when it is lane-agnostic: each
    consumer can rebuild it from the primary it already loads."""
    return _is_lane_agnostic(elem)


def try_prologue_absorb_multi(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """Single-op elem read by 2+ vertices, every one an anchor vertex whose
    load boundary includes it: copy the elem into each; drop the original
    when nothing else reads it."""
    for v in graph.vertices:
        if not _is_elementwise_vertex(v) or len(v.ops) != 1:
            continue
        elem = v.ops[0]
        if not (_prologue_eligible(elem) and _should_recompute(elem)):
            continue
        name = elem.out.name
        if name not in v.outputs:
            continue
        readers = graph.consumers_of(name)
        if len(readers) < 2:
            continue
        anchor_ids: list[int] = []
        for r in readers:
            anc = _anchor_of(r)
            if anc is None or name not in _anchor_boundary_input_names(anc, r):
                break
            anchor_ids.append(id(anc))
        else:
            sig = v.op_ids | frozenset(oid for r in readers for oid in r.op_ids)
            if sig in blacklist:
                continue
            g = graph
            for aid in anchor_ids:
                target = next(cv for cv in g.vertices if any(id(op) == aid for op in cv.ops))
                g = g.absorb_into(target, v.ops)
            still_read = name in graph.program_outputs or any(
                name in other.inputs for other in g.vertices if other is not v
            )
            return g if still_read else g.remove_vertex(v)
    return None


_PASSES = (
    try_elem_chain_fuse,
    try_multi_producer_chain_fuse,  # extension, off unless MULTI_ANCHOR_MERGE_CHAINS
    try_multi_producer_fuse,  # must precede epilogue absorption (it would steal the merge)
    try_epilogue_absorb,
    try_prologue_absorb_single,
    try_prologue_absorb_multi,
)


# Extension beyond the reference's rules, off by default: a last-axis
# reduction of a matmul's output (after the matmul's lane-agnostic register
# epilogue, with no prologue) is computed by the matmul's kernel, which
# writes the matmul output and the reduction both.  C5's S = Q @ K^T * s and
# m1 = max(S) become one kernel, so S is not read back for m1.  It runs on
# the reference's saturated partition (the reference's passes never see a
# vertex holding both), and the reduction vertex must be the reduction alone.
MATMUL_REDUCTION_EPILOGUES = False
_ROW_REDUCTIONS = ("sum", "max", "min", "product")


def try_matmul_reduction_fuse(graph: Graph, blacklist: Blacklist) -> Graph | None:
    """(Extension, ``MATMUL_REDUCTION_EPILOGUES``.)  A vertex holding one
    reduction whose input is the last output of a vertex holding one matmul
    as its first op and lane-agnostic elementwise ops after it."""
    if not MATMUL_REDUCTION_EPILOGUES:
        return None
    for r in graph.vertices:
        if len(r.ops) != 1 or not isinstance(r.ops[0], ReductionOp) or r.ops[0].op not in _ROW_REDUCTIONS:
            continue
        red = r.ops[0]
        a = graph.producer_of(red.input.name)
        if a is None or a is r or not isinstance(a.ops[0], MatmulOp) or a.ops[-1].out.name != red.input.name:
            continue
        if not all(isinstance(op, ElementwiseOp) and _is_lane_agnostic(op) for op in a.ops[1:]):
            continue
        if (a.op_ids | r.op_ids) in blacklist:
            continue
        return graph.replace(absorbed=(a, r), ops=_by_position(graph, (*a.ops, *r.ops)))
    return None


# Extension passes, tried in order on the reference's saturated partition.
_LATE_PASSES = (try_matmul_reduction_fuse,)


# ---------------------------------------------------------------------------
# Budget gate and driver (reference: fusion.py:443-545)
# ---------------------------------------------------------------------------


def _cap() -> int:
    # Read the module global at call time so tests can monkeypatch it.
    return globals()["TGMEM_CAP_BYTES"]


def _budget_bytes(vertex: Vertex) -> int:
    from metellus_amd.orchestrator.assembly import assemble

    return compute_group_budget(assemble(vertex)).size_bytes


def _check_primitive_budgets(graph: Graph) -> None:
    cap = _cap()
    for v in graph.vertices:
        need = _budget_bytes(v)
        if need > cap:
            names = ", ".join(f"{type(op).__name__}({op.out.name})" for op in v.ops)
            raise TgmemOverflowError(
                f"primitive vertex [{names}] needs {need}B of LDS; cap is {cap}B. "
                "No fusion can shrink a single op — reduce its tile shape or pick "
                "a register-resident strategy."
            )


def _new_vertices(old: Graph, new: Graph) -> list[Vertex]:
    seen = {id(v) for v in old.vertices}
    return [v for v in new.vertices if id(v) not in seen]


def _fits_budget(old: Graph, new: Graph) -> bool:
    cap = _cap()
    return all(_budget_bytes(v) <= cap for v in _new_vertices(old, new))


def _modified_signature(old: Graph, new: Graph) -> frozenset[int]:
    sig: frozenset[int] = frozenset()
    for v in _new_vertices(old, new):
        sig = sig | v.op_ids
    return sig


def _fuse_once(program: Program, blacklist: Blacklist) -> tuple[tuple[Vertex, ...], frozenset[int] | None]:
    graph = Graph.from_program(program)
    _check_primitive_budgets(graph)
    for passes in (_PASSES, _LATE_PASSES):
        while True:
            for rewrite in passes:
                candidate = rewrite(graph, blacklist)
                if candidate is None:
                    continue
                if not _fits_budget(graph, candidate):
                    return candidate.topo_sort(), _modified_signature(graph, candidate)
                graph = candidate
                break
            else:
                break
    return graph.topo_sort(), None


def fuse(program: Program) -> tuple[Vertex, ...]:
    """Saturate the passes; on an over-budget rewrite, blacklist it and
    rerun from the primitive graph.  Deterministic."""
    blacklist: frozenset[frozenset[int]] = frozenset()
    while True:
        vertices, straw = _fuse_once(program, blacklist)
        if straw is None:
            return vertices
        blacklist = blacklist | {straw}
