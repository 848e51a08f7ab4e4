"""``mt_div_fast`` (division where the quotient enters a matmul) against
IEEE division on the GPU: within 1 ulp for every finite pair, identical
(NaN matching NaN) where an operand or the result is zero, subnormal, huge,
infinite or NaN (those take the IEEE path)."""

import numpy as np
import pytest

from metellus_amd.compute.fragments import device_header
from metellus_amd.runtime import hip_backend
from metellus_amd.runtime.buffer import Buffer

pytestmark = pytest.mark.gpu

_SRC = device_header() + r"""
extern "C" __global__ void __launch_bounds__(256)
div_pair(const float* __restrict__ x, const float* __restrict__ y, float* __restrict__ fast,
         float* __restrict__ ieee, const mt_dims dims) {
    const unsigned i = blockIdx.x * 256u + threadIdx.x;
    if (i < dims.v[0]) {
        fast[i] = mt_div_fast(x[i], y[i]);
        ieee[i] = x[i] / y[i];
    }
}
"""


def _ulp_distance(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_fast_division_matches_ieee():
    rng = np.random.default_rng(31)
    n = 1 << 22
    x = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))).astype(np.float32)
    y = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-42, 1e-38, 3e38, -3e38, 1.0, -2.5],
                       dtype=np.float32)
    sx, sy = np.meshgrid(special, special)
    x[: sx.size] = sx.ravel()
    y[: sy.size] = sy.ravel()
    bx, by, bf, bi = Buffer.from_numpy(x), Buffer.from_numpy(y), Buffer(n * 4), Buffer(n * 4)
    kernel = hip_backend.compile_kernel(_SRC, "div_pair")
    hip_backend.launch(kernel, [bx, by, bf, bi], (n,), 4, ((n + 255) // 256, 1, 1), (256, 1, 1))
    fast, ieee = bf.numpy((n,), np.float32), bi.numpy((n,), np.float32)
    for b in (bx, by, bf, bi):
        b.release()
    np.testing.assert_array_equal(ieee, x / y)  # the device division is IEEE
    edge = ~(np.isfinite(x) & np.isfinite(y) & np.isfinite(ieee)) | (np.abs(y) < 2.0 ** -125) \
        | (np.abs(y) > 2.0 ** 125) | (np.abs(ieee) > 2.0 ** 124)
    np.testing.assert_array_equal(fast[edge], ieee[edge])
    normal = ~edge & (np.abs(ieee) > 2.0 ** -126)  # quotients in the normal range
    d = _ulp_distance(fast[normal], ieee[normal])
    assert d.max() <= 1, f"max ulp distance {d.max()}"
    exact = float(np.mean(d == 0))
    print(f"mt_div_fast: {exact:.6%} of {normal.sum()} normal quotients exact, max 1 ulp")
    assert exact > 0.99
    # subnormal quotients: within float32 absolute resolution there
    sub = ~edge & ~normal
    assert np.all(np.abs(fast[sub].astype(np.float64) - ieee[sub]) <= 2.0 ** -148)
