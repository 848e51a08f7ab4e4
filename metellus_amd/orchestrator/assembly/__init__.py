"""Assemble a fused ``Vertex`` into a ``KernelGroup`` (reference:
src/orchestrator/assembly/__init__.py:59-74): classify, then dispatch to the
strategy's template."""

from __future__ import annotations

from metellus_amd.orchestrator.assembly.decision import classify
from metellus_amd.orchestrator.assembly.elementwise import assemble_elementwise
from metellus_amd.orchestrator.assembly.matmul import assemble_matmul
from metellus_amd.orchestrator.assembly.multi_anchor import assemble_multi_anchor
from metellus_amd.orchestrator.assembly.reduction import assemble_reduction
from metellus_amd.orchestrator.assembly.shape import assemble_shape
from metellus_amd.orchestrator.graph import Vertex
from metellus_amd.orchestrator.kernel_group import FusionStrategy, KernelGroup

_MATMUL = {
    FusionStrategy.STANDALONE_MATMUL,
    FusionStrategy.MATMUL_EPILOGUE_TG,
    FusionStrategy.MATMUL_EPILOGUE_REGISTER,
    FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
    FusionStrategy.MATMUL_REDUCTION_EPILOGUE,
}
_REDUCTION = {
    FusionStrategy.STANDALONE_REDUCTION,
    FusionStrategy.REDUCTION_EPILOGUE,
    FusionStrategy.ELEMENTWISE_PROLOGUE_REDUCTION,
}
_ELEMENTWISE = {FusionStrategy.STANDALONE_ELEMENTWISE, FusionStrategy.ELEMENTWISE_CHAIN}
_MULTI = {FusionStrategy.MULTI_PRODUCER_CONVERGENT, FusionStrategy.DIAMOND_SHARED}


def assemble(vertex: Vertex, *, function_name: str | None = None, batch: int = 1) -> KernelGroup:
    """``batch`` > 1: the kernel will be launched for that many identical
    programs at once (``Kernel.batched``); matmul tiles are chosen for the
    combined grid."""
    decision = classify(vertex)
    s = decision.strategy
    if s in _MATMUL:
        return assemble_matmul(decision, function_name, batch=batch)
    if s in _REDUCTION:
        return assemble_reduction(decision, function_name)
    if s in _ELEMENTWISE:
        return assemble_elementwise(decision, function_name)
    if s is FusionStrategy.STANDALONE_SHAPE:
        return assemble_shape(decision, function_name)
    if s in _MULTI:
        return assemble_multi_anchor(decision, function_name, batch=batch)
    raise ValueError(f"unknown strategy {s!r}")


__all__ = ["assemble"]
