"""``metal_backend.run_kernel`` through the reference's module name, with the
reference's three kinds of slot (reference: src/metal_backend.mm:153-176):
a ``Buffer``, an int handle, and a NumPy array, which is uploaded to a
one-shot device buffer and, after the kernel, copied back into the array
(reference: src/metal_backend.mm:235-239).  The kernels are the
hand-composed ones of ``tests/fragment_kernels.py``; results are checked
against the oracle: exactly for IEEE-exact ops and copies, and at the matmul
bar for the GEMM."""

from __future__ import annotations

import numpy as np
import pytest

import metellus_amd

metellus_amd.install_reference_namespace()

import metal_backend  # noqa: E402  (the reference's native module name)
from oracle.ir_eval import BINARY, matmul_tolerance  # noqa: E402
from runtime import Buffer  # noqa: E402
from tests import fragment_kernels as fk  # noqa: E402

pytestmark = pytest.mark.gpu


def test_reference_name_is_the_hip_backend():
    from metellus_amd.runtime import hip_backend

    assert metal_backend is hip_backend and metal_backend.run_kernel is hip_backend.run_kernel


def test_buffer_and_array_slots_elementwise():
    """X as a Buffer, Y and Out as arrays: Out receives the kernel's result,
    Y comes back unchanged, X's buffer is untouched."""
    metal_backend.init()
    rng = np.random.default_rng(51)
    M, N = 37, 45
    x = rng.standard_normal((M, N)).astype(np.float32)
    y = rng.standard_normal((M, N)).astype(np.float32)
    kernel, bindings, dims, grid, threads = fk.elementwise_kernel("add", M, N, y.shape)
    assert bindings == ("X", "Y", "Out")
    xb = Buffer.from_numpy(x)
    y_arr = y.copy()
    out = np.full((M, N), np.nan, dtype=np.float32)
    before = metal_backend.alloc_stats()["live_buffers"]
    res = metal_backend.run_kernel(kernel.source, kernel.function_name, [xb, y_arr, out], grid, threads,
                                   dims=dims, dims_slot=kernel.dims_slot_index)
    assert set(res) == {"time_ms"} and isinstance(res["time_ms"], float) and res["time_ms"] > 0.0
    np.testing.assert_array_equal(out, BINARY["add"](x, y))
    np.testing.assert_array_equal(y_arr, y)
    np.testing.assert_array_equal(xb.numpy((M, N), np.float32), x)
    # the one-shot buffers are gone again
    assert metal_backend.alloc_stats()["live_buffers"] == before
    xb.release()


def test_int_handle_buffer_and_array_slots_gemm():
    """A as an int handle, B as a Buffer, C as an array (ragged shape: the
    LDS C-tile path of the hand-composed GEMM)."""
    metal_backend.init()
    rng = np.random.default_rng(52)
    m, k, n = 100, 70, 130
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    kernel, tile, aligned, grid = fk.gemm_kernel(m, k, n)
    assert not aligned
    threads = (tile.tg_x, tile.tg_y, 1)
    h = metal_backend.create_buffer(a.nbytes)
    metal_backend.write_buffer(h, a)
    bb = Buffer.from_numpy(b)
    c = np.full((m, n), np.nan, dtype=np.float32)
    res = metal_backend.run_kernel(kernel.source, kernel.function_name, [h, bb, c], grid, threads,
                                   dims=(m, k, n), dims_slot=kernel.dims_slot_index)
    assert res["time_ms"] > 0.0
    err = np.abs(c.astype(np.float64) - a.astype(np.float64) @ b.astype(np.float64))
    assert not np.isnan(c).any()
    assert np.all(err <= matmul_tolerance(a, b) + 1e-30), f"max err {err.max():.3e}"
    metal_backend.release_buffer(h)
    bb.release()


def test_array_slots_written_back_in_order():
    """Every array slot is written back after the kernel, in slot order: a
    copy kernel reading one array and writing another leaves the input array
    as it was and the output array equal to it.  A zero-size array binds a
    valid (unused) pointer."""
    metal_backend.init()
    n = 4097
    src = np.linspace(-3.0, 3.0, n, dtype=np.float32)
    src_arr = src.copy()
    out = np.zeros(n, dtype=np.float32)
    kernel = fk.copy_kernel()
    res = metal_backend.run_kernel(kernel.source, kernel.function_name, [out, src_arr], fk.init_grid(n),
                                   (fk.TG_X, 1, 1), dims=(n,), dims_slot=kernel.dims_slot_index)
    assert res["time_ms"] > 0.0
    np.testing.assert_array_equal(out, src)
    np.testing.assert_array_equal(src_arr, src)
    # the same kernel over 0 elements: nothing is launched on the arrays' data
    empty_out, empty_in = np.zeros(0, np.float32), np.zeros(0, np.float32)
    metal_backend.run_kernel(kernel.source, kernel.function_name, [empty_out, empty_in], (1, 1, 1),
                             (fk.TG_X, 1, 1), dims=(0,), dims_slot=kernel.dims_slot_index)
    assert empty_out.size == 0
