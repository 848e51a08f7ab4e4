"""``KernelGroup``: one generated kernel plus everything needed to launch it
(reference: src/orchestrator/kernel_group.py:1-82).  Strategy names and
values are the reference's, so callers can introspect fusion plans the
same way."""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

from metellus_amd.orchestrator.ir import Op
from metellus_amd.runtime.program import Kernel


class FusionStrategy(str, Enum):
    STANDALONE_MATMUL = "standalone_matmul"
    STANDALONE_ELEMENTWISE = "standalone_elementwise"
    STANDALONE_REDUCTION = "standalone_reduction"
    MATMUL_EPILOGUE_REGISTER = "matmul_epilogue_register"
    MATMUL_EPILOGUE_TG = "matmul_epilogue_tg"
    ELEMENTWISE_PROLOGUE_MATMUL = "elementwise_prologue_matmul"
    ELEMENTWISE_PROLOGUE_REDUCTION = "elementwise_prologue_reduction"
    REDUCTION_EPILOGUE = "reduction_epilogue"
    ELEMENTWISE_CHAIN = "elementwise_chain"
    STANDALONE_SHAPE = "standalone_shape"
    MULTI_PRODUCER_CONVERGENT = "multi_producer_convergent"
    DIAMOND_SHARED = "diamond_shared"
    # extension (fusion.MATMUL_REDUCTION_EPILOGUES): a matmul whose output
    # also feeds a last-axis reduction computed in the same kernel
    MATMUL_REDUCTION_EPILOGUE = "matmul_reduction_epilogue"

    def __str__(self) -> str:
        return self.value


@dataclass(frozen=True)
class KernelGroup:
    """``bindings``: env keys in kernel-parameter order; ``dims``: runtime
    values for ``kernel.ctx.dims``; ``grid``: workgroups per axis;
    ``threads``: lanes per workgroup; ``ops``: IR ops fused in, in IR order."""

    kernel: Kernel
    bindings: tuple[str, ...]
    dims: tuple[int, ...]
    grid: tuple[int, int, int]
    threads: tuple[int, int, int]
    ops: tuple[Op, ...]
    strategy: FusionStrategy

    @property
    def outputs(self) -> tuple[str, ...]:
        return tuple(op.out.name for op in self.ops if op.out.name in self.bindings)
