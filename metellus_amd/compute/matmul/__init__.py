from metellus_amd.compute.matmul.matmul import (
    MatmulAccumToDevFragment,
    MatmulComputeFragment,
    MatmulConfig,
    MatmulEpilogueStoreFragment,
    MatmulMainloopFragment,
    MatmulRegisterEpilogueFragment,
    MatmulSetupFragment,
    MatmulTileMappingFragment,
    ThreadIndexFragment,
)

__all__ = [
    "MatmulAccumToDevFragment",
    "MatmulComputeFragment",
    "MatmulConfig",
    "MatmulEpilogueStoreFragment",
    "MatmulMainloopFragment",
    "MatmulRegisterEpilogueFragment",
    "MatmulSetupFragment",
    "MatmulTileMappingFragment",
    "ThreadIndexFragment",
]
