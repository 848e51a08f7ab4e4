"""End-to-end compile + run (reference: src/api/run.py:25-40):
``ops.build() -> fuse -> assemble -> alias_group -> schedule -> Runtime.run()``."""

from __future__ import annotations

from typing import Any, NamedTuple

from metellus_amd.orchestrator.aliasing import alias_group
from metellus_amd.orchestrator.assembly import assemble
from metellus_amd.orchestrator.builder import Operations
from metellus_amd.orchestrator.fusion import fuse
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.orchestrator.scheduler import schedule


class RunResult(NamedTuple):
    env: dict[str, Any]
    groups: tuple[KernelGroup, ...]


def compile_program(ops: Operations) -> tuple[KernelGroup, ...]:
    """The four host stages, without executing anything."""
    return tuple(alias_group(assemble(v)) for v in fuse(ops.build()))


def run(ops: Operations, *, profile: bool = False) -> RunResult:
    """Compile and execute; outputs land in ``env`` under their tensor names
    (``profile=True`` adds per-kernel GPU ms as ``t_0``, ``t_1``, ...)."""
    groups = compile_program(ops)
    runtime = schedule(ops, groups, profile=profile)
    return RunResult(env=runtime.run(), groups=groups)
