"""Runtime: packed-weight store and the device kernels."""
from .store import PackedModelStore, PackedWeight

__all__ = ["PackedModelStore", "PackedWeight"]
