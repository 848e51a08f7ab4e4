"""The reference's fragment-level benches (tests/bench_init.py,
bench_reduction.py, bench_elementwise.py, bench_matmul.py) compose kernels
by hand.  Without a GPU: every such kernel renders with this package's
fragments and compiles for gfx950; the loaders pick safe access modes when
strides and limits are symbolic.  Their results are GPU tests
(``test_gpu_fragment_suites.py``)."""

import pytest

from metellus_amd.runtime import hip_backend
from tests import fragment_kernels as fk


def _compiles(kernel):
    assert hip_backend.compile_only(kernel.source) > 0


@pytest.mark.parametrize("make", [lambda: fk.fill_kernel(3.5), lambda: fk.arange_kernel(-2.0, 0.5), fk.copy_kernel])
def test_init_kernels_compile(make):
    _compiles(make())


def test_init_rejects_non_finite_literals():
    with pytest.raises(ValueError, match="non-finite"):
        fk.fill_kernel(float("inf")).source


@pytest.mark.parametrize("op", ["sum", "max", "min", "product"])
def test_reduction_kernels_compile_with_symbolic_row_length(op):
    k = fk.reduction_kernel(op)
    src = k.source
    assert "mt_ld4" not in src.split('extern "C"')[1]  # N is symbolic: per-element loads
    _compiles(k)


@pytest.mark.parametrize("op", fk.UNARY_OPS + fk.BINARY_OPS + ["where"])
def test_elementwise_kernels_compile(op):
    from compute.elementwise import elementwise_arity

    n = elementwise_arity(op)
    k, *_ = fk.elementwise_kernel(op, 10, 13, (10, 13) if n >= 2 else None, (10, 13) if n == 3 else None)
    body = k.source.split('extern "C"')[1]
    assert "fetch_safe(" in body  # row strides are run-time dims
    assert "(threadIdx.y * 32u + threadIdx.x)" in body  # 32 x 8 workgroups
    _compiles(k)


@pytest.mark.parametrize("shape", fk.GEMM_SHAPES)
def test_gemm_kernels_compile(shape):
    k, tile, aligned, grid = fk.gemm_kernel(*shape)
    body = k.source.split('extern "C"')[1]
    assert ("C_tile" in body) == (not aligned)
    assert "sizeof(A_tile[0]) / sizeof(float)" in body  # pitch of the declared (padded) tile
    _compiles(k)
