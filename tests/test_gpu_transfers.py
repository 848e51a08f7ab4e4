"""Host <-> device transfers through the shim.  Large transfers from or to
pageable memory go through a ring of page-locked staging buffers in 16 MiB
chunks; page-locked memory and small transfers copy directly.  Every path
must move the bytes exactly: sizes around the direct/staged threshold
(4 MiB) and the chunk size, partial reads, and a write ordered after a
kernel still queued on the stream."""

from __future__ import annotations

import ctypes
import time

import numpy as np
import pytest

from metellus_amd.runtime import hip_backend
from metellus_amd.runtime.buffer import Buffer

pytestmark = pytest.mark.gpu

MIB = 1 << 20
SIZES = [4, 4 * MIB - 4, 4 * MIB, 16 * MIB - 4, 16 * MIB, 16 * MIB + 4, 48 * MIB + 12, 100 * MIB + 4]


def _pattern(nbytes: int, seed: int) -> np.ndarray:
    # distinct words everywhere, so a misplaced chunk cannot go unnoticed
    rng = np.random.default_rng(seed)
    return (np.arange(nbytes // 4, dtype=np.uint32) * np.uint32(2654435761) + np.uint32(rng.integers(1 << 31))).view(
        np.uint32
    )


@pytest.mark.parametrize("nbytes", SIZES)
def test_round_trip_pageable_and_pinned(nbytes):
    src = _pattern(nbytes, nbytes)
    buf = Buffer.from_numpy(src)  # pageable source
    back = np.empty_like(src)  # pageable destination
    hip_backend.read_buffer(buf.handle, back)
    np.testing.assert_array_equal(back, src)
    pinned = buf.numpy(src.shape, np.uint32)  # page-locked pool block when >= 1 MiB
    np.testing.assert_array_equal(pinned, src)
    buf.release()


def test_partial_read_and_overwrite():
    n = 40 * MIB
    a, b = _pattern(n, 1), _pattern(n, 2)
    buf = Buffer.from_numpy(a)
    head = np.empty(17 * MIB // 4 + 3, dtype=np.uint32)
    hip_backend.read_buffer(buf.handle, head)
    np.testing.assert_array_equal(head, a[: head.size])
    buf.write(b)
    back = np.empty_like(b)
    hip_backend.read_buffer(buf.handle, back)
    np.testing.assert_array_equal(back, b)


def test_write_after_queued_kernel_is_stream_ordered():
    """A fill queued before a large pageable write must not land after it."""
    n = 32 * MIB
    buf = Buffer(n)
    buf.fill(0xAB)  # stream-ordered memset, not synchronised
    src = _pattern(n, 3)
    hip_backend.write_buffer(buf.handle, src)
    back = np.empty_like(src)
    hip_backend.read_buffer(buf.handle, back)
    np.testing.assert_array_equal(back, src)


def test_transfer_rates_reported():
    """Not a bar: prints the measured rates (they are quoted in the design notes)."""
    n = 256 * MIB
    src = np.random.default_rng(0).standard_normal(n // 4).astype(np.float32)
    buf = Buffer(n)
    dst = np.empty_like(src)
    lib = hip_backend.library()
    rates = {}
    for name, fn in (
        ("H2D pageable", lambda: hip_backend.write_buffer(buf.handle, src)),
        ("D2H pageable", lambda: lib.mt_read(buf.handle, dst.ctypes.data_as(ctypes.c_void_p), n)),
    ):
        fn()
        t = min(_timed(fn) for _ in range(3))
        rates[name] = n / t / 1e9
    np.testing.assert_array_equal(dst, src)
    print({k: round(v, 1) for k, v in rates.items()})


def _timed(fn) -> float:
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0
