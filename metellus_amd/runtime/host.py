"""Host arrays backed by page-locked memory from the shim's pinned pool.

A device-to-host copy into page-locked memory runs at the link's DMA rate
and touches no fresh pages, where a copy into a new pageable NumPy array
pays the runtime's staging copy and a page fault per 4 KiB.  Large
downloads therefore land in ``pinned_empty`` arrays: ordinary NumPy arrays
whose memory goes back to the pool when the last reference to them is
dropped.
"""

from __future__ import annotations

import atexit
import ctypes

import numpy as np

from metellus_amd.runtime import hip_backend

PINNED_MIN_BYTES = 1 << 20  # smaller downloads use ordinary arrays

_shutting_down = False


def _mark_shutdown() -> None:
    global _shutting_down
    _shutting_down = True


atexit.register(_mark_shutdown)


class _PinnedBlock:
    """Owns one pooled block; returns it to the pool when collected."""

    __slots__ = ("address", "__weakref__")

    def __init__(self, nbytes: int) -> None:
        self.address = hip_backend.host_alloc(nbytes)

    def __del__(self) -> None:
        if self.address and not _shutting_down:
            try:
                hip_backend.host_free(self.address)
            except Exception:
                pass
        self.address = 0


def pinned_empty(shape: tuple[int, ...], dtype) -> np.ndarray:
    """An uninitialised C-contiguous array in page-locked memory."""
    dtype = np.dtype(dtype)
    count = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    nbytes = max(1, count * dtype.itemsize)
    block = _PinnedBlock(nbytes)
    raw = (ctypes.c_char * nbytes).from_address(block.address)
    raw._owner = block  # the ctypes view keeps the block alive; the array keeps the view
    return np.frombuffer(raw, dtype=dtype, count=count).reshape(shape)
