"""``Buffer``: owning handle to a device allocation in the shim's registry
(reference: src/runtime/buffer.py:8-91).  Freed by ``release()`` or when the
object is collected; frees are stream-ordered, so a kernel already queued
on the buffer still sees it."""

from __future__ import annotations

import numpy as np

from metellus_amd.runtime import hip_backend


class Buffer:
    __slots__ = ("_handle", "_nbytes", "_released")

    def __init__(self, nbytes: int) -> None:
        if nbytes <= 0:
            raise ValueError(f"Buffer nbytes must be > 0; got {nbytes}")
        self._released = True  # until the allocation succeeds
        self._handle = hip_backend.create_buffer(nbytes)
        self._nbytes = int(nbytes)
        self._released = False

    @classmethod
    def from_numpy(cls, array: np.ndarray) -> "Buffer":
        dense = np.ascontiguousarray(array)
        buf = cls(dense.nbytes)
        hip_backend.write_buffer(buf._handle, dense)
        return buf

    @classmethod
    def zeros(cls, nbytes: int) -> "Buffer":
        buf = cls(nbytes)
        hip_backend.fill_buffer(buf._handle, 0)
        return buf

    @property
    def handle(self) -> int:
        if self._released:
            raise RuntimeError("Buffer has been released")
        return self._handle

    @property
    def nbytes(self) -> int:
        return self._nbytes

    @property
    def device_address(self) -> int:
        return hip_backend.device_address(self.handle)

    def write(self, array: np.ndarray) -> None:
        dense = np.ascontiguousarray(array)
        if dense.nbytes > self._nbytes:
            raise ValueError(f"write: source ({dense.nbytes} bytes) exceeds buffer ({self._nbytes} bytes)")
        hip_backend.write_buffer(self.handle, dense)

    def read_into(self, out: np.ndarray) -> np.ndarray:
        if not out.flags["C_CONTIGUOUS"]:
            raise ValueError("read_into: destination must be C-contiguous")
        if out.nbytes > self._nbytes:
            raise ValueError(f"read_into: destination ({out.nbytes} bytes) exceeds buffer ({self._nbytes} bytes)")
        hip_backend.read_buffer(self.handle, out)
        return out

    def numpy(self, shape: tuple[int, ...], dtype) -> np.ndarray:
        """Download into a new array (page-locked from the pinned pool when
        it is at least ``PINNED_MIN_BYTES``)."""
        from metellus_amd.runtime.host import PINNED_MIN_BYTES, pinned_empty

        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        out = pinned_empty(shape, dtype) if nbytes >= PINNED_MIN_BYTES else np.empty(shape, dtype=dtype)
        return self.read_into(out)

    def fill(self, byte_value: int) -> None:
        if not 0 <= byte_value <= 255:
            raise ValueError(f"fill byte_value must be in [0, 255]; got {byte_value}")
        hip_backend.fill_buffer(self.handle, byte_value)

    def release(self) -> None:
        if not self._released:
            self._released = True
            hip_backend.release_buffer(self._handle)

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass

    def __repr__(self) -> str:
        state = "released" if self._released else f"handle={self._handle}"
        return f"Buffer(nbytes={self._nbytes}, {state})"
