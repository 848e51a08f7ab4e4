"""Orchestrator: IR, builder, DAG and vertex graph.  ``fuse``, ``assemble``,
``schedule``, ``KernelGroup`` and ``FusionStrategy`` live in their
submodules (as in the reference, src/orchestrator/__init__.py)."""

from metellus_amd.compute.elementwise.elementwise import BroadcastSpec
from metellus_amd.orchestrator.builder import Operations
from metellus_amd.orchestrator.dag import DAG, build_dag
from metellus_amd.orchestrator.graph import Graph, Vertex
from metellus_amd.orchestrator.ir import (
    ElementwiseOp,
    Layout,
    MatmulOp,
    Op,
    OperandValue,
    Program,
    ReductionOp,
    Scalar,
    ShapeOp,
    Tensor,
)

__all__ = [
    "BroadcastSpec",
    "DAG",
    "ElementwiseOp",
    "Graph",
    "Layout",
    "MatmulOp",
    "Op",
    "OperandValue",
    "Operations",
    "Program",
    "ReductionOp",
    "Scalar",
    "ShapeOp",
    "Tensor",
    "Vertex",
    "build_dag",
]
