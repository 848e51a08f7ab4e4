from metellus_amd.memory.memory import TgLoadFragment, TgStoreFragment, ValueTransform

__all__ = ["TgLoadFragment", "TgStoreFragment", "ValueTransform"]
