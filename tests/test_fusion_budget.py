"""The LDS budget gate of ``fuse`` (the reference's
tests/test_fusion_budget.py, re-derived for gfx950 tiles).

gfx950 numbers used below (64x64x32 MFMA tile for 64x64 operands,
double-buffered).  A single matmul and the diamond load their operand tiles
straight into dense LDS tiles: one matmul = A 2x64x32 + B 2x32x64 floats =
32,768 B; the diamond (shared A, two B chunks) = 49,152 B.  The non-shared
multi-producer fills registers-first tiles with padded rows (A rows of 36
floats, B rows of 68): 35,840 B, because its second mainloop's tiles alias
the first's.  The real cap is 163,840 B."""

import pytest

from orchestrator import Operations
from orchestrator.aliasing import TGMEM_CAP_BYTES, TgmemOverflowError, compute_group_budget
from orchestrator.assembly import assemble
from orchestrator.fusion import fuse
from orchestrator.kernel_group import FusionStrategy


def _budget(v) -> int:
    return compute_group_budget(assemble(v)).size_bytes


def _pair(shared: bool, n: int = 64):
    ops = Operations()
    ops.input("A", shape=(n, n))
    if shared:
        ops.input("B1", shape=(n, n))
        ops.input("B2", shape=(n, n))
        ops.matmul(a="A", b="B1", out="c1")
        ops.matmul(a="A", b="B2", out="c2")
    else:
        for name in "BCD":
            ops.input(name, shape=(n, n))
        ops.matmul(a="A", b="B", out="c1")
        ops.matmul(a="C", b="D", out="c2")
    ops.elementwise("add", out="z", operands=("c1", "c2"))
    return ops


def test_cap_is_gfx950_lds():
    assert TGMEM_CAP_BYTES == 163_840


def test_fits_under_cap_unchanged():
    ops = Operations()
    ops.input("A", shape=(32, 64))
    ops.input("B", shape=(64, 128))
    ops.input("bias", shape=(1, 128))
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("add", out="Cb", operands=("C", "bias"), y_broadcast="row")
    ops.elementwise("max", out="y", operands=("Cb", 0.0))
    (v,) = fuse(ops.build())
    assert _budget(v) <= TGMEM_CAP_BYTES


def test_budget_numbers():
    (d,) = fuse(_pair(True).build())
    (m,) = fuse(_pair(False).build())
    assert _budget(d) == 49_152
    assert _budget(m) == 35_840  # A1/B1 alias A0/B0
    ops = Operations()
    ops.input("A", shape=(64, 64))
    ops.input("B", shape=(64, 64))
    ops.matmul(a="A", b="B", out="C")
    (p,) = fuse(ops.build())
    assert _budget(p) == 32_768


def test_overflowing_fusion_is_blacklisted_and_split(monkeypatch):
    monkeypatch.setattr("orchestrator.fusion.TGMEM_CAP_BYTES", 45_056)
    vs = fuse(_pair(True).build())
    assert len(vs) > 1
    for v in vs:
        assert _budget(v) <= 45_056
    groups = sorted(tuple(sorted(type(op).__name__ for op in v.ops)) for v in vs)
    assert ("MatmulOp",) in groups


def test_aliasing_lets_multi_producer_fit_where_diamond_cannot(monkeypatch):
    monkeypatch.setattr("orchestrator.fusion.TGMEM_CAP_BYTES", 45_056)
    (v,) = fuse(_pair(False).build())
    assert assemble(v).strategy is FusionStrategy.MULTI_PRODUCER_CONVERGENT


def test_irreducible_primitive_raises(monkeypatch):
    monkeypatch.setattr("orchestrator.fusion.TGMEM_CAP_BYTES", 64)
    ops = Operations()
    ops.input("A", shape=(32, 32))
    ops.input("B", shape=(32, 32))
    ops.matmul(a="A", b="B", out="C")
    with pytest.raises(TgmemOverflowError) as err:
        fuse(ops.build())
    assert "MatmulOp" in str(err.value) and "C" in str(err.value)


def test_blacklist_retry_is_deterministic(monkeypatch):
    monkeypatch.setattr("orchestrator.fusion.TGMEM_CAP_BYTES", 45_056)
    a = fuse(_pair(True).build())
    b = fuse(_pair(True).build())
    assert [[type(op).__name__ for op in v.ops] for v in a] == [[type(op).__name__ for op in v.ops] for v in b]
