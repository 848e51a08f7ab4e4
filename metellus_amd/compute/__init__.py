"""HIP fragment library for gfx950 (device half: ``csrc/mt_device.h``)."""

from metellus_amd.compute.fragments import (
    AliasFragment,
    BarrierFragment,
    CodegenContext,
    CodegenEngine,
    TgmemAccess,
)

__all__ = ["AliasFragment", "BarrierFragment", "CodegenContext", "CodegenEngine", "TgmemAccess"]
