"""The shim's device block cache: released buffers stay with the shim and
serve later allocations of their size class, in stream order, until
``trim`` hands them back to the driver."""

from __future__ import annotations

import gc

import numpy as np
import pytest

from metellus_amd.runtime import hip_backend
from metellus_amd.runtime.buffer import Buffer

pytestmark = pytest.mark.gpu

MIB = 1 << 20

# y[i] = 2 x[i] + 1 over n floats (n = dims.v[0]); grid covers n exactly.
_TWICE = r"""
struct dc_dims { unsigned int v[16]; };
extern "C" __global__ void __launch_bounds__(256)
twice(const float* __restrict__ x, float* __restrict__ y, const dc_dims d) {
    const unsigned i = blockIdx.x * 256u + threadIdx.x;
    if (i < d.v[0]) y[i] = 2.0f * x[i] + 1.0f;
}
"""


def _clean():
    gc.collect()  # buffers of earlier tests still waiting for their finaliser
    hip_backend.trim()


def test_released_block_is_reused_and_trimmed():
    _clean()
    assert hip_backend.device_cache_info() == (0, 0)
    a = Buffer(256 * MIB)
    addr = a.device_address
    a.release()
    assert hip_backend.device_cache_info() == (256 * MIB, 1)
    b = Buffer(256 * MIB - 3 * MIB)  # same size class within 1/8: the cached block
    assert b.device_address == addr and hip_backend.device_cache_info() == (0, 0)
    src = np.arange(b.nbytes // 4, dtype=np.uint32)
    b.write(src)
    np.testing.assert_array_equal(b.numpy(src.shape, np.uint32), src)
    c = Buffer(128 * MIB)  # smaller than 7/8 of the block: a new allocation
    b.release()
    d = Buffer(100 * MIB)  # the 256 MiB block is too big for it: new
    assert d.device_address != addr
    assert hip_backend.device_cache_info() == (256 * MIB, 1)  # the block keeps its size class
    for x in (c, d):
        x.release()
    hip_backend.trim()
    assert hip_backend.device_cache_info() == (0, 0)


def test_small_blocks_round_to_256_bytes():
    _clean()
    a = Buffer(1000)
    addr = a.device_address
    a.release()
    assert hip_backend.device_cache_info() == (1024, 1)
    b = Buffer(1024)
    assert b.device_address == addr
    b.release()
    hip_backend.trim()


def test_reuse_is_ordered_after_queued_kernels():
    """A kernel reading x is queued, x is released and its block handed to a
    new buffer that is overwritten at once: the kernel still sees x's data."""
    n = 64 * MIB // 4
    kernel = hip_backend.compile_kernel(_TWICE, "twice")
    x0 = np.random.default_rng(0).standard_normal(n).astype(np.float32)
    x = Buffer.from_numpy(x0)
    y = Buffer(4 * n)
    _clean()
    for _ in range(4):  # queue a few launches so the release lands while they run
        hip_backend.launch(kernel, [x, y], [n], 2, (n // 256, 1, 1), (256, 1, 1))
    addr = x.device_address
    x.release()
    z = Buffer(4 * n)
    assert z.device_address == addr
    z.write(np.full(n, 7.0, dtype=np.float32))  # staged copy on the same stream
    np.testing.assert_array_equal(y.numpy((n,), np.float32), 2.0 * x0 + 1.0)
    np.testing.assert_array_equal(z.numpy((n,), np.float32), np.full(n, 7.0, dtype=np.float32))
    for b in (y, z):
        b.release()
    hip_backend.trim()
