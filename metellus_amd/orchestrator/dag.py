"""Flat producer/consumer view of a Program (reference:
src/orchestrator/dag.py:1-76).  Validates SSA and definition-before-use."""

from __future__ import annotations

from dataclasses import dataclass

from metellus_amd.orchestrator.ir import Op, Program


@dataclass(frozen=True)
class DAG:
    program: Program
    producer_of: dict[str, Op]
    consumers_of: dict[str, tuple[Op, ...]]
    inputs: frozenset[str]
    outputs: frozenset[str]

    def unique_consumer(self, name: str) -> Op | None:
        readers = self.consumers_of.get(name, ())
        return readers[0] if len(readers) == 1 else None

    def topo_order(self) -> list[Op]:
        """The program is already in topological order; returns a copy."""
        return list(self.program)


def build_dag(program: Program) -> DAG:
    producer_of: dict[str, Op] = {}
    readers: dict[str, list[Op]] = {}
    for op in program:
        for t in op.inputs:
            readers.setdefault(t.name, []).append(op)
        name = op.out.name
        if name in producer_of:
            raise ValueError(f"SSA violation: tensor {name!r} produced by two ops")
        if name in readers:
            raise ValueError(
                f"def-after-use: tensor {name!r} consumed before it is defined "
                "(program must be in topological order)"
            )
        producer_of[name] = op
    used = set(readers)
    produced = set(producer_of)
    return DAG(
        program=list(program),
        producer_of=producer_of,
        consumers_of={k: tuple(v) for k, v in readers.items()},
        inputs=frozenset(used - produced),
        outputs=frozenset(produced - used),
    )
