from metellus_amd.compute.reduction.reduction import (
    REDUCTION_OPS,
    LastAxisReductionComputeFragment,
    LastAxisReductionSetupFragment,
    StoreReductionResultFragment,
    ValueTransform,
)

__all__ = [
    "LastAxisReductionComputeFragment",
    "LastAxisReductionSetupFragment",
    "REDUCTION_OPS",
    "StoreReductionResultFragment",
    "ValueTransform",
]
