from metellus_amd.compute.copy.copy import StridedCopyFragment

__all__ = ["StridedCopyFragment"]
