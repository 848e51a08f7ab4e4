from metellus_amd.compute.elementwise.elementwise import (
    BROADCAST_MODES,
    BroadcastSpec,
    ElementwiseComputeFragment,
    elementwise_arity,
    elementwise_compute_block,
    elementwise_expression,
    elementwise_outputs_bool,
    elementwise_threadgroup_section,
    supported_elementwise_ops,
)

__all__ = [
    "BROADCAST_MODES",
    "BroadcastSpec",
    "ElementwiseComputeFragment",
    "elementwise_arity",
    "elementwise_compute_block",
    "elementwise_expression",
    "elementwise_outputs_bool",
    "elementwise_threadgroup_section",
    "supported_elementwise_ops",
]
