"""End-to-end compile + run (reference: src/api/run.py:25-40):
``ops.build() -> fuse -> assemble -> alias_group -> schedule -> Runtime.run()``.

``run_batch`` runs several programs of identical structure (e.g. the 32
attention heads of one layer, each a 2-D program) together: each fused
kernel is launched once for all programs (grid z = program index, buffers
passed as per-program pointer tables), instead of once per program."""

from __future__ import annotations

from collections.abc import Iterable

from typing import Any, NamedTuple

import numpy as np

from metellus_amd.orchestrator.aliasing import alias_group
from metellus_amd.orchestrator.assembly import assemble
from metellus_amd.orchestrator.builder import Operations
from metellus_amd.orchestrator.fusion import fuse
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.orchestrator.scheduler import schedule
from metellus_amd.runtime.program import Dispatch, Runtime


class RunResult(NamedTuple):
    env: dict[str, Any]
    groups: tuple[KernelGroup, ...]


def compile_program(ops: Operations, *, batch: int = 1) -> tuple[KernelGroup, ...]:
    """The four host stages, without executing anything."""
    return tuple(alias_group(assemble(v, batch=batch)) for v in fuse(ops.build()))


def run(ops: Operations, *, profile: bool = False, outputs: Iterable[str] | None = None) -> RunResult:
    """Compile and execute; outputs land in ``env`` under their tensor names
    (``profile=True`` adds per-kernel GPU ms as ``t_0``, ``t_1``, ...).
    ``outputs`` limits the downloads to those names (every materialised
    tensor otherwise, as in the reference)."""
    groups = compile_program(ops)
    runtime = schedule(ops, groups, profile=profile, outputs=outputs)
    return RunResult(env=runtime.run(), groups=groups)


def _same_plan(plans: list[Runtime]) -> bool:
    first = plans[0].fragments
    for rt in plans[1:]:
        if len(rt.fragments) != len(first):
            return False
        for a, b in zip(first, rt.fragments):
            if type(a) is not type(b):
                return False
            if isinstance(a, Dispatch) and (
                a.kernel.source != b.kernel.source
                or a.bindings != b.bindings
                or a.dims != b.dims
                or a.grid != b.grid
                or a.threads != b.threads
            ):
                return False
    return True


class BatchRunner:
    """Executes the schedules of ``len(programs)`` structurally identical
    programs in lockstep; every Dispatch is one batched launch."""

    def __init__(
        self, programs: list[Operations], *, profile: bool = False, outputs: Iterable[str] | None = None
    ) -> None:
        self.programs = list(programs)
        self.groups = [compile_program(ops, batch=len(self.programs)) for ops in self.programs]
        outputs = None if outputs is None else tuple(outputs)
        self.plans = [
            schedule(ops, g, profile=profile, outputs=outputs) for ops, g in zip(self.programs, self.groups)
        ]
        self.batched = len(self.programs) > 1 and _same_plan(self.plans)

    def run(self) -> list[RunResult]:
        from metellus_amd.runtime import hip_backend
        from metellus_amd.runtime.buffer import Buffer

        envs: list[dict] = [{} for _ in self.programs]
        if not self.batched:
            for rt, env in zip(self.plans, envs):
                rt.run(env)
            return [RunResult(env=e, groups=g) for e, g in zip(envs, self.groups)]
        B = len(self.programs)
        for steps in zip(*(rt.fragments for rt in self.plans)):
            head = steps[0]
            if not isinstance(head, Dispatch):
                for step, env in zip(steps, envs):
                    step.execute(env)
                continue
            tables = []
            for key in head.bindings:
                addrs = np.array([env[key].device_address for env in envs], dtype=np.uint64)
                tables.append(Buffer.from_numpy(addrs))
            kernel = head.kernel.batched()
            ms = hip_backend.launch(
                kernel.handle,
                tables,
                head.dims,
                kernel.dims_slot_index,
                (head.grid[0], head.grid[1], head.grid[2] * B),
                head.threads,
                timed=head.time_key is not None,
                workspace=kernel.workspace_bytes,
            )
            if head.time_key is not None:
                for env in envs:
                    env[head.time_key] = float(ms)
            del tables  # stream-ordered frees: safe after the launch is queued
        return [RunResult(env=e, groups=g) for e, g in zip(envs, self.groups)]


def run_batch(
    programs: list[Operations], *, profile: bool = False, outputs: Iterable[str] | None = None
) -> list[RunResult]:
    """Run structurally identical programs with one launch per fused kernel
    for the whole batch (falls back to one run per program when their plans
    differ).  With ``profile`` each env gets the batched launch time;
    ``outputs`` limits the downloads as in ``run``."""
    return BatchRunner(programs, profile=profile, outputs=outputs).run()
