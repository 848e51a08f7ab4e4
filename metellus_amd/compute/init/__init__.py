from metellus_amd.compute.init.init import ArangeFragment, CopyFragment, FillFragment

__all__ = ["ArangeFragment", "CopyFragment", "FillFragment"]
