"""Vertex graph: the rewrite substrate the fuser works on.

Behaviour follows the reference (src/orchestrator/graph.py:1-428): a
``Graph`` is a DAG of ``Vertex``es (each holding 1+ IR ops in program order
plus an input/output boundary); ``replace`` collapses a convex vertex set,
``absorb_into`` replicates producer ops into a consumer (multi-consumer
recompute), ``topo_sort`` orders vertices deterministically by the earliest
contained op's program position, and ``check_dependencies`` verifies a
rewritten graph against the original program.

Views (transpose / reshape) are not graph nodes; a consumer of a view sees
the view's name as an external input.  Ordering between a view's owner and
its consumers therefore comes only from the position tie-break
(reference: graph.py:21-24).

Implementation notes (behaviour-neutral): the topological order and the
producer map of an immutable graph are computed once and cached, and the
order is produced with a heap keyed by (earliest op position, vertex
position) instead of re-sorting a list after every pop.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass
from functools import cached_property

from metellus_amd.orchestrator.ir import Op, Program


@dataclass(frozen=True)
class Vertex:
    """1+ IR ops in program order with the tensors read from outside
    (``inputs``) and the tensors written for outside readers (``outputs``)."""

    ops: tuple[Op, ...]
    inputs: tuple[str, ...]
    outputs: tuple[str, ...]

    @property
    def is_primitive(self) -> bool:
        return len(self.ops) == 1

    @property
    def op_ids(self) -> frozenset[int]:
        return frozenset(id(op) for op in self.ops)


@dataclass(frozen=True)
class Graph:
    vertices: tuple[Vertex, ...]
    op_index: dict[int, int]
    program_outputs: frozenset[str]

    # -- construction --------------------------------------------------------

    @classmethod
    def from_program(cls, program: Program, *, program_outputs: frozenset[str] | None = None) -> Graph:
        """One vertex per op.  ``program_outputs`` defaults to the sinks
        (produced, never read).  A vertex exports its tensor iff something
        reads it or it is a program output."""
        read: set[str] = {t.name for op in program for t in op.inputs}
        made: set[str] = {op.out.name for op in program}
        outs = frozenset(made - read) if program_outputs is None else frozenset(program_outputs)
        verts = []
        for op in program:
            name = op.out.name
            exported = (name,) if (name in read or name in outs) else ()
            verts.append(Vertex(ops=(op,), inputs=tuple(t.name for t in op.inputs), outputs=exported))
        return cls(
            vertices=tuple(verts),
            op_index={id(op): i for i, op in enumerate(program)},
            program_outputs=outs,
        )

    def _derive(self, vertices: tuple[Vertex, ...]) -> Graph:
        return Graph(vertices=vertices, op_index=self.op_index, program_outputs=self.program_outputs)

    # -- cached structure ----------------------------------------------------

    @cached_property
    def _producers(self) -> dict[str, Vertex]:
        """tensor name -> first vertex exporting it (vertex order)."""
        found: dict[str, Vertex] = {}
        for v in self.vertices:
            for name in v.outputs:
                found.setdefault(name, v)
        return found

    @cached_property
    def _order(self) -> tuple[Vertex, ...] | None:
        """Deterministic topological order, or None when cyclic."""
        # Edges follow the *last* exporter of a name, like a dict overwrite.
        writer: dict[str, int] = {}
        for pos, v in enumerate(self.vertices):
            for name in v.outputs:
                writer[name] = pos
        n = len(self.vertices)
        succ: list[set[int]] = [set() for _ in range(n)]
        indeg = [0] * n
        for pos, v in enumerate(self.vertices):
            preds = {writer[name] for name in v.inputs if name in writer}
            indeg[pos] = len(preds)
            for p in preds:
                succ[p].add(pos)
        key = [min(self.op_index[id(op)] for op in v.ops) for v in self.vertices]
        heap = [(key[p], p) for p in range(n) if indeg[p] == 0]
        heapq.heapify(heap)
        order: list[int] = []
        while heap:
            _, p = heapq.heappop(heap)
            order.append(p)
            for s in succ[p]:
                indeg[s] -= 1
                if indeg[s] == 0:
                    heapq.heappush(heap, (key[s], s))
        if len(order) != n:
            return None
        return tuple(self.vertices[p] for p in order)

    # -- queries -------------------------------------------------------------

    def topo_sort(self) -> tuple[Vertex, ...]:
        order = self._order
        if order is None:
            raise ValueError("graph contains a cycle")
        return order

    def flatten(self) -> tuple[Op, ...]:
        return tuple(op for v in self.topo_sort() for op in v.ops)

    def producer_of(self, name: str) -> Vertex | None:
        return self._producers.get(name)

    def consumers_of(self, name: str) -> tuple[Vertex, ...]:
        """Vertices reading ``name``, in topological order."""
        return tuple(v for v in self.topo_sort() if name in v.inputs)

    def check_dependencies(self, original: Program) -> None:
        """Every producer->consumer edge of ``original`` must be honoured by
        ``flatten()``: each position of a consumer op has some position of
        its producer op before it (ops replicated by ``absorb_into`` occur
        several times)."""
        flat = self.flatten()
        where: dict[int, list[int]] = {}
        for i, op in enumerate(flat):
            where.setdefault(id(op), []).append(i)
        orig_ids = {id(op) for op in original}
        missing = [op for op in original if id(op) not in where]
        if missing:
            names = [f"{type(op).__name__}({op.out.name})" for op in missing]
            raise ValueError(f"graph missing IR ops: {names}")
        if set(where) - orig_ids:
            raise ValueError(
                "graph contains ops not in original IR — replace() received "
                "ops that don't belong to this Program"
            )
        made_by = {op.out.name: op for op in original}
        for op in original:
            for t in op.inputs:
                prod = made_by.get(t.name)
                if prod is None:
                    continue
                first_prod = min(where[id(prod)])
                for pos in where[id(op)]:
                    if first_prod >= pos:
                        raise ValueError(
                            f"dependency violated: {type(prod).__name__}({prod.out.name}) "
                            f"has no occurrence before {type(op).__name__}({op.out.name}) "
                            f"at flatten-pos {pos} (consumed via tensor {t.name!r})"
                        )

    def preserves_dependencies(self, original: Program) -> bool:
        try:
            self.check_dependencies(original)
        except ValueError:
            return False
        return True

    # -- rewrites ------------------------------------------------------------

    def replace(self, absorbed: tuple[Vertex, ...], ops: tuple[Op, ...]) -> Graph:
        """Collapse ``absorbed`` into one vertex holding ``ops`` (their union,
        in program order).  New inputs = absorbed inputs minus names made
        inside; new outputs = names made inside that a surviving vertex reads
        or that are program outputs.  The new vertex takes the position of
        the first absorbed vertex.  Raises if the collapse creates a cycle
        (reference: graph.py:118-212)."""
        if not absorbed:
            raise ValueError("replace: absorbed set is empty")
        present = {id(v) for v in self.vertices}
        taken: set[int] = set()
        for v in absorbed:
            if id(v) not in present:
                raise ValueError("replace: absorbed contains a vertex not in this graph")
            if id(v) in taken:
                raise ValueError("replace: absorbed contains duplicate vertices")
            taken.add(id(v))
        if frozenset(id(op) for v in absorbed for op in v.ops) != frozenset(id(op) for op in ops):
            raise ValueError("replace: ops does not match the union of absorbed vertices' ops")
        positions = [self.op_index[id(op)] for op in ops]
        if positions != sorted(positions):
            raise ValueError("replace: ops must be in original-IR program order")

        made = {op.out.name for op in ops}
        read_outside: set[str] = set()
        for v in self.vertices:
            if id(v) not in taken:
                read_outside.update(v.inputs)
        read_inside: set[str] = set()
        for v in absorbed:
            read_inside.update(v.inputs)
        merged = Vertex(
            ops=tuple(ops),
            inputs=tuple(sorted(read_inside - made)),
            outputs=tuple(sorted(n for n in made if n in read_outside or n in self.program_outputs)),
        )
        new_vertices: list[Vertex] = []
        placed = False
        for v in self.vertices:
            if id(v) not in taken:
                new_vertices.append(v)
            elif not placed:
                new_vertices.append(merged)
                placed = True
        result = self._derive(tuple(new_vertices))
        if result._order is None:
            raise ValueError(
                "replace: collapsing the absorbed set would introduce a cycle — "
                "the absorbed vertices are not convex in the dependency order"
            )
        return result

    def absorb_into(self, consumer: Vertex, additional_ops: tuple[Op, ...]) -> Graph:
        """Copy ``additional_ops`` into ``consumer`` (merged by program
        position); the producing vertex is left in place
        (reference: graph.py:335-390)."""
        if all(v is not consumer for v in self.vertices):
            raise ValueError("absorb_into: consumer not in this graph")
        if not additional_ops:
            raise ValueError("absorb_into: additional_ops is empty")
        merged_ops = tuple(
            sorted((*additional_ops, *consumer.ops), key=lambda op: self.op_index[id(op)])
        )
        extra_in = {t.name for op in additional_ops for t in op.inputs}
        extra_out = {op.out.name for op in additional_ops}
        grown = Vertex(
            ops=merged_ops,
            inputs=tuple(sorted((set(consumer.inputs) | extra_in) - extra_out)),
            outputs=consumer.outputs,
        )
        result = self._derive(tuple(grown if v is consumer else v for v in self.vertices))
        if result._order is None:
            raise ValueError(
                "absorb_into: result is cyclic (additional_ops' inputs "
                "transitively depend on the consumer's outputs)"
            )
        return result

    def remove_vertex(self, vertex: Vertex) -> Graph:
        """Drop a vertex whose outputs nobody reads and which exports no
        program output."""
        if all(v is not vertex for v in self.vertices):
            raise ValueError("remove_vertex: vertex not in this graph")
        for name in vertex.outputs:
            if name in self.program_outputs:
                raise ValueError(f"remove_vertex: output {name!r} is a program output; cannot remove")
            if any(other is not vertex and name in other.inputs for other in self.vertices):
                raise ValueError(f"remove_vertex: output {name!r} still consumed by another vertex")
        return self._derive(tuple(v for v in self.vertices if v is not vertex))
