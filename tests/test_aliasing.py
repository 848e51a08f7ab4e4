"""LDS lifetime analysis, slot packing and the alias rewrite.

The packing rule (reference: src/orchestrator/aliasing.py:209-289) is fully
specified, so these tests check hand-computed plans: a lifetime joins a
slot whose last tenant died strictly before it is born, choosing least
growth, then smallest slot, then most recent death."""

import pytest

from orchestrator import Operations
from orchestrator.aliasing import (
    AliasFragment,
    TgmemLifetime,
    alias_group,
    compute_alias_map,
    compute_budget,
    compute_lifetimes,
)
from orchestrator.assembly import assemble
from orchestrator.fusion import fuse


def _lt(name, b, d, size):
    return TgmemLifetime(name=name, birth=b, death=d, size_floats=size, shape=(size,))


def test_empty_plan():
    assert compute_alias_map(()).slots == ()


def test_overlapping_lifetimes_get_separate_slots():
    plan = compute_alias_map((_lt("a", 0, 3, 100), _lt("b", 1, 2, 50)))
    assert [s.tenants for s in plan.slots] == [("a",), ("b",)]
    assert plan.total_size_floats == 150


def test_disjoint_lifetimes_share_and_slot_grows_to_largest():
    plan = compute_alias_map((_lt("a", 0, 1, 100), _lt("b", 2, 3, 300)))
    (slot,) = plan.slots
    assert slot.tenants == ("a", "b") and slot.size_floats == 300 and slot.name == "a"
    assert plan.name_to_slot == {"a": "a", "b": "a"}


def test_prefers_zero_growth_then_tightest_slot():
    # c (size 40, born at 4) can join x (200) or y (50): both free, both fit
    # -> tightest fit y.  d (size 180, born 5): only x is free (y now holds c
    # until 6) -> x.
    lts = (_lt("x", 0, 1, 200), _lt("y", 0, 2, 50), _lt("c", 4, 6, 40), _lt("d", 5, 7, 180))
    plan = compute_alias_map(lts)
    assert [s.tenants for s in plan.slots] == [("x", "d"), ("y", "c")]
    assert plan.total_size_floats == 250
    assert compute_budget(lts).size_bytes == 1000


def test_least_growth_wins_over_size():
    # e (size 120, born 3) can go to p (100, growth 20) or q (60, growth 60)
    plan = compute_alias_map((_lt("p", 0, 1, 100), _lt("q", 0, 2, 60), _lt("e", 3, 4, 120)))
    assert [s.tenants for s in plan.slots] == [("p", "e"), ("q",)]
    assert plan.total_size_floats == 180


def test_touching_lifetimes_do_not_share():
    plan = compute_alias_map((_lt("a", 0, 2, 10), _lt("b", 2, 3, 10)))
    assert len(plan.slots) == 2


def _multi_producer():
    ops = Operations()
    for name in "ABCD":
        ops.input(name, shape=(64, 64))
    ops.matmul(a="A", b="B", out="c1")
    ops.matmul(a="C", b="D", out="c2")
    ops.elementwise("add", out="z", operands=("c1", "c2"))
    return assemble(fuse(ops.build())[0])


def test_multi_producer_lifetimes_and_rewrite():
    g = _multi_producer()
    lts = {lt.name: lt for lt in compute_lifetimes(g.kernel)}
    assert lts["A0_tile"].birth == lts["A0_tile"].death < lts["A1_tile"].birth
    aliased = alias_group(g)
    decls = aliased.kernel.ctx.threadgroup_decls
    assert len(decls) == 2 and all("_storage[" in d for d in decls)
    aliases = [f for f in aliased.kernel.fragments if isinstance(f, AliasFragment)]
    assert {a.new_name for a in aliases} == {"A0_tile", "B0_tile", "A1_tile", "B1_tile"}
    # the second tenants need a barrier after the first mainloop
    late = [a for a in aliases if a.new_name in ("A1_tile", "B1_tile")]
    assert any(not a.preceded_by_barrier for a in late)
    src = aliased.kernel.source
    assert "float (*A1_tile)[64][36] = reinterpret_cast<float (*)[64][36]>(_A0_tile_storage);" in src


def test_single_tenant_kernels_are_unchanged():
    ops = Operations()
    ops.input("A", shape=(64, 64))
    ops.input("B", shape=(64, 64))
    ops.matmul(a="A", b="B", out="C")
    g = assemble(fuse(ops.build())[0])
    assert alias_group(g).kernel.ctx.threadgroup_decls == g.kernel.ctx.threadgroup_decls


def test_unparseable_declaration_rejected():
    import dataclasses

    from orchestrator.aliasing import apply_alias_map

    g = _multi_producer()
    bad_ctx = dataclasses.replace(g.kernel.ctx, threadgroup_decls=("float A0_tile[4];",))
    from runtime import Kernel

    k = Kernel(g.kernel.fragments, bad_ctx)
    with pytest.raises(ValueError, match="cannot parse"):
        apply_alias_map(k, compute_alias_map(compute_lifetimes(k)))


def _with_c_tile(persistent_capacity, monkeypatch):
    """An assembled matmul with a C tile staged through LDS after its
    mainloop (MatmulAccumToTgFragment -> barrier -> MatmulTgToDevFragment),
    as a hand-composed kernel would add it."""
    import dataclasses

    from compute.fragments import BarrierFragment, lds_decl
    from compute.matmul import config
    from compute.matmul.matmul import (
        MatmulAccumToTgFragment,
        MatmulEpilogueStoreFragment,
        MatmulMainloopFragment,
        MatmulTgToDevFragment,
    )
    from runtime import Kernel

    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", persistent_capacity)
    monkeypatch.setattr(config, "STREAM_K", False)
    ops = Operations()
    ops.input("A", shape=(512, 256))
    ops.input("B", shape=(256, 512))
    ops.matmul(a="A", b="B", out="C")
    g = assemble(fuse(ops.build())[0])
    frags = list(g.kernel.fragments)
    i = next(k for k, f in enumerate(frags) if isinstance(f, MatmulEpilogueStoreFragment))
    cfg = next(f for f in frags if isinstance(f, MatmulMainloopFragment)).fragments[3].config
    frags[i : i + 1] = [MatmulAccumToTgFragment(cfg), BarrierFragment("c_ready"), MatmulTgToDevFragment(cfg)]
    t = cfg.tile
    decls = (*g.kernel.ctx.threadgroup_decls, lds_decl("C_tile", (t.tile_M, t.tile_N + t.c_pad)))
    return Kernel(tuple(frags), dataclasses.replace(g.kernel.ctx, threadgroup_decls=decls))


def test_persistent_loop_keeps_post_mainloop_tenants_apart(monkeypatch):
    # In a persistent tile loop the mainloop's last chunk loads the next
    # tile's first chunk into A_tile/B_tile (directly into LDS) while the
    # epilogue runs, so a C tile born after the mainloop must not reuse
    # their storage.
    k = _with_c_tile(2, monkeypatch)
    assert any(getattr(f, "opens_tile_loop", False) for f in k.fragments)
    plan = compute_alias_map(compute_lifetimes(k))
    slot_of = plan.name_to_slot
    assert slot_of["C_tile"] not in (slot_of["A_tile"], slot_of["B_tile"])
    assert all(len(s.tenants) == 1 for s in plan.slots)
    lts = {lt.name: lt for lt in compute_lifetimes(k)}
    end = next(i for i, f in enumerate(k.fragments) if getattr(f, "closes_tile_loop", False))
    assert lts["A_tile"].death == end and lts["C_tile"].death == end


def test_one_tile_per_workgroup_lets_the_c_tile_reuse_operand_storage(monkeypatch):
    # the same kernel without the loop: straight-line code, so the C tile
    # (born after the operands' last use) joins an operand slot
    k = _with_c_tile(10_000, monkeypatch)
    assert not any(getattr(f, "opens_tile_loop", False) for f in k.fragments)
    plan = compute_alias_map(compute_lifetimes(k))
    assert any("C_tile" in s.tenants and len(s.tenants) > 1 for s in plan.slots)
