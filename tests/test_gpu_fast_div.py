"""``mt_div_fast`` (division where the quotient enters a matmul) against
IEEE division on the GPU.  Divisors with 1 <= |y| < 2^125 take the
refined-reciprocal product: within 2 ulp, and identical for zero, infinite
and NaN numerators.  Divisors with 2^-125 < |y| < 1 add one residual
correction: within 1 ulp.  Zero, subnormal, huge and non-finite divisors
(and huge quotients of small divisors) take the IEEE path: identical, NaN
matching NaN."""

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
    ay = np.abs(y)
    ieee_path = ~np.isfinite(y) | (ay <= 2.0 ** -125) | (ay >= 2.0 ** 125) | ~np.isfinite(x) \
        | ((ay < 1.0) & (np.abs(ieee) > 2.0 ** 126))
    np.testing.assert_array_equal(fast[ieee_path], ieee[ieee_path])
    finite = ~ieee_path & np.isfinite(ieee)
    product = finite & (ay >= 1.0)
    corrected = finite & (ay < 1.0)
    normal = np.abs(ieee) > 2.0 ** -126  # quotients in the normal range
    d_prod = _ulp_distance(fast[product & normal], ieee[product & normal])
    d_corr = _ulp_distance(fast[corrected & normal], ieee[corrected & normal])
    assert d_prod.max() <= 2, f"product path: max ulp distance {d_prod.max()}"
    assert d_corr.max() <= 1, f"corrected path: max ulp distance {d_corr.max()}"
    exact_prod, exact_corr = float(np.mean(d_prod == 0)), float(np.mean(d_corr == 0))
    print(f"mt_div_fast: product path {exact_prod:.4%} exact of {d_prod.size} (max {d_prod.max()} ulp); "
          f"corrected path {exact_corr:.4%} exact of {d_corr.size}")
    assert exact_prod > 0.6 and exact_corr > 0.99
    # zero numerators keep their sign on the product path; subnormal
    # quotients stay within float32's absolute resolution there
    zero = product & (x == 0)
    np.testing.assert_array_equal(fast[zero].view(np.uint32), ieee[zero].view(np.uint32))
    sub = finite & ~normal
    assert np.all(np.abs(fast[sub].astype(np.float64) - ieee[sub]) <= 2.0 ** -148)


@pytest.mark.parametrize("op", ["div", "recip"])
def test_fused_epilogue_division_rounds_like_the_unfused_chain(op):
    """A division fused into a matmul's register epilogue is IEEE division,
    so ``(A @ B) / d`` and ``recip(A @ B)`` fused give exactly what the same
    op gives in its own elementwise kernel on the matmul's output."""
    from metellus_amd.api import run
    from metellus_amd.orchestrator import Operations

    rng = np.random.default_rng(37)
    a = rng.standard_normal((256, 192)).astype(np.float32)
    b = rng.standard_normal((192, 320)).astype(np.float32)
    d = rng.uniform(0.3, 3.0, 256).astype(np.float32)

    def tail(ops, src):
        if op == "div":
            ops.from_numpy(d, "d")
            ops.reshape("d", (256, 1), out="dc")
            ops.elementwise("div", out="Y", operands=(src, "dc"), y_broadcast="col")
        else:
            ops.elementwise("recip", out="Y", operands=(src,))

    fused = Operations()
    fused.from_numpy(a, "A")
    fused.from_numpy(b, "B")
    fused.matmul(a="A", b="B", out="C")
    tail(fused, "C")
    res = run(fused, outputs=("Y",))
    assert len(res.groups) == 1, [g.strategy for g in res.groups]
    assert "mt_div_fast(" not in "".join(res.groups[0].kernel.ctx.helpers)
    mm = Operations()
    mm.from_numpy(a, "A")
    mm.from_numpy(b, "B")
    mm.matmul(a="A", b="B", out="C")
    c = run(mm).env["C"]
    ew = Operations()
    ew.from_numpy(c, "Cm")
    tail(ew, "Cm")
    unfused = run(ew).env["Y"]
    np.testing.assert_array_equal(res.env["Y"], unfused)


@pytest.mark.parametrize("divisors", ["plain", "some rows not plain"])
def test_plain_commit_matches_per_element_division(divisors, monkeypatch):
    """Y = (E / s[row]) @ V with the divisor gathered per row: the commit
    that tests every divisor once per wave and then multiplies by 1/s
    (``commit_apply_fast``) gives the bits of the per-element
    ``mt_div_fast`` commit -- also when some rows' divisors (below 1, zero,
    subnormal, infinite) send their waves down the per-element path."""
    from metellus_amd.api import run
    from metellus_amd.orchestrator import Operations
    from metellus_amd.orchestrator.assembly import matmul as mm

    rng = np.random.default_rng(41)
    M, K, N = 512, 256, 128
    e = rng.random((M, K), dtype=np.float32) + 0.1
    s = (rng.random(M, dtype=np.float32) * 100.0 + 1.0).astype(np.float32)
    if divisors != "plain":
        s[[3, 77, 130, 400, 401]] = np.array([0.5, 0.0, 1e-40, np.inf, 2.0 ** 126], dtype=np.float32)
    v = rng.standard_normal((K, N)).astype(np.float32)

    def program():
        ops = Operations()
        ops.from_numpy(e, "E")
        ops.from_numpy(s, "s")
        ops.from_numpy(v, "V")
        ops.reshape("s", (M, 1), out="sv")
        ops.elementwise("div", out="P", operands=("E", "sv"), y_broadcast="col")
        ops.matmul(a="P", b="V", out="Y")
        return ops

    outs = {}
    for plain in (True, False):
        monkeypatch.setattr(mm, "PLAIN_COMMIT", plain)
        res = run(program(), outputs=("Y",))
        src = res.groups[0].kernel.source.split('extern "C"')[-1]
        assert ("commit_apply_fast<" in src) == plain
        outs[plain] = res.env["Y"]
    np.testing.assert_array_equal(outs[True], outs[False])
