"""LDS lifetime analysis, slot aliasing and the fusion budget.

Algorithm and API follow the reference (src/orchestrator/aliasing.py:1-490):

1. ``compute_lifetimes`` walks the kernel's top-level fragments (recursing
   into ``sub_fragments``) and records, per LDS name, the first and last
   top-level index touching it and its largest footprint.
2. ``compute_alias_map`` packs lifetimes into slots greedily in birth order:
   a lifetime may join a slot whose last tenant died strictly before it is
   born; among those it picks the least growth, then the smallest slot,
   then the most recently freed; otherwise it opens a slot.
3. ``apply_alias_map`` replaces the declarations of every multi-tenant slot
   by one flat ``__shared__`` storage array and re-types it per tenant with
   a pointer alias, placed after the latest barrier in the gap between the
   previous tenant's death and the new tenant's birth (or with its own
   barrier when the gap has none).

The budget the fuser gates on is the sum of slot sizes -- exactly the LDS
the rewritten kernel declares.  The cap is gfx950's static LDS limit per
workgroup, 163,840 bytes (160 KiB; 163,844 bytes is rejected by the
compiler), in place of the reference's 32 KiB Apple limit (:44).
"""

from __future__ import annotations

import dataclasses
import re
from dataclasses import dataclass
from typing import Iterable

from metellus_amd.compute.fragments import AliasFragment, TgmemAccess, lds_decl
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel

TGMEM_CAP_BYTES = 163_840
"""Static LDS per workgroup on gfx950 (MI355X)."""


class TgmemOverflowError(RuntimeError):
    """A kernel's LDS plan cannot fit under ``TGMEM_CAP_BYTES``."""


@dataclass(frozen=True)
class TgmemLifetime:
    name: str
    birth: int
    death: int
    size_floats: int
    shape: tuple[int, ...]


def _walk_accesses(fragment: object) -> Iterable[TgmemAccess]:
    yield from getattr(fragment, "tgmem_accesses", ())
    for sub in getattr(fragment, "sub_fragments", ()):
        yield from _walk_accesses(sub)


def _tile_loops(kernel: Kernel) -> list[tuple[int, int]]:
    """(open, close) top-level indices of the persistent tile loops: a
    fragment with ``opens_tile_loop`` true up to the next one with
    ``closes_tile_loop``."""
    spans, start = [], None
    for idx, frag in enumerate(kernel.fragments):
        if getattr(frag, "opens_tile_loop", False):
            start = idx
        elif getattr(frag, "closes_tile_loop", False) and start is not None:
            spans.append((start, idx))
            start = None
    if start is not None:
        raise ValueError("a persistent tile loop is opened but never closed")
    return spans


def compute_lifetimes(kernel: Kernel) -> tuple[TgmemLifetime, ...]:
    """One lifetime per LDS name, in first-touch order.

    The fragments are straight-line code except inside a persistent tile
    loop, where the last k-chunk of an item already loads the next item's
    first chunk into the operand tiles (directly into LDS, possibly still in
    flight) while the item's epilogue runs: every name touched inside such a
    loop lives for the whole loop, so nothing touched there shares a slot
    with anything else touched there."""
    first: dict[str, int] = {}
    last: dict[str, int] = {}
    biggest: dict[str, TgmemAccess] = {}
    for idx, frag in enumerate(kernel.fragments):
        for acc in _walk_accesses(frag):
            if acc.name not in first:
                first[acc.name] = idx
                biggest[acc.name] = acc
            elif acc.size_floats > biggest[acc.name].size_floats:
                biggest[acc.name] = acc
            last[acc.name] = idx
    for lo, hi in _tile_loops(kernel):
        for n in first:
            if first[n] <= hi and last[n] >= lo:
                first[n], last[n] = min(first[n], lo), max(last[n], hi)
    return tuple(
        TgmemLifetime(
            name=n,
            birth=first[n],
            death=last[n],
            size_floats=biggest[n].size_floats,
            shape=tuple(biggest[n].shape),
        )
        for n in first
    )


def compute_group_lifetimes(group: KernelGroup) -> tuple[TgmemLifetime, ...]:
    return compute_lifetimes(group.kernel)


@dataclass(frozen=True)
class FusionBudget:
    """Static LDS footprint of one kernel after aliasing."""

    n_slots: int
    size_floats: int

    @property
    def size_bytes(self) -> int:
        return 4 * self.size_floats


@dataclass(frozen=True)
class AliasSlot:
    name: str
    tenants: tuple[str, ...]
    size_floats: int
    shape: tuple[int, ...]


@dataclass(frozen=True)
class AliasMap:
    slots: tuple[AliasSlot, ...]

    @property
    def name_to_slot(self) -> dict[str, str]:
        return {t: s.name for s in self.slots for t in s.tenants}

    @property
    def total_size_floats(self) -> int:
        return sum(s.size_floats for s in self.slots)

    @property
    def n_slots(self) -> int:
        return len(self.slots)


def compute_alias_map(lifetimes: tuple[TgmemLifetime, ...]) -> AliasMap:
    """Birth-order greedy packing (reference: aliasing.py:209-289)."""
    tenants: list[list[TgmemLifetime]] = []
    size: list[int] = []
    for lt in sorted(lifetimes, key=lambda t: (t.birth, t.death)):
        choice = None
        choice_key = None
        for i, slot in enumerate(tenants):
            prev = slot[-1]
            if prev.death >= lt.birth:
                continue
            growth = max(0, lt.size_floats - size[i])
            rank = (growth, size[i], -prev.death)
            if choice_key is None or rank < choice_key:
                choice, choice_key = i, rank
        if choice is None:
            tenants.append([lt])
            size.append(lt.size_floats)
        else:
            tenants[choice].append(lt)
            size[choice] = max(size[choice], lt.size_floats)
    return AliasMap(
        slots=tuple(
            AliasSlot(name=ts[0].name, tenants=tuple(t.name for t in ts), size_floats=sz, shape=ts[0].shape)
            for ts, sz in zip(tenants, size)
        )
    )


def compute_budget(lifetimes: tuple[TgmemLifetime, ...]) -> FusionBudget:
    plan = compute_alias_map(lifetimes)
    return FusionBudget(n_slots=plan.n_slots, size_floats=plan.total_size_floats)


def compute_group_budget(group: KernelGroup) -> FusionBudget:
    return compute_budget(compute_lifetimes(group.kernel))


def compute_group_alias_map(group: KernelGroup) -> AliasMap:
    return compute_alias_map(compute_lifetimes(group.kernel))


# Canonical declaration: `__shared__ [alignas(N)] float <name>[d]...;`
_DECL_RE = re.compile(
    r"^\s*__shared__\s+(?:alignas\(\s*\d+\s*\)\s+)?float\s+(\w+)\s*(?:\[[^\]]+\])+\s*;\s*$"
)


def _decl_name(decl: str) -> str:
    m = _DECL_RE.match(decl)
    if m is None:
        raise ValueError(
            f"apply_alias_map: cannot parse LDS declaration {decl!r}. "
            "Expected `__shared__ [alignas(N)] float <name>[N]...;`."
        )
    return m.group(1)


def _is_barrier(fragment: object) -> bool:
    return getattr(fragment, "is_tgmem_barrier", False) is True


def _storage_name(owner: str) -> str:
    return f"_{owner}_storage"


def apply_alias_map(kernel: Kernel, alias_map: AliasMap) -> Kernel:
    """Rewrite ``kernel`` so every multi-tenant slot shares one storage array
    (reference: aliasing.py:340-453)."""
    if not alias_map.slots:
        return kernel
    by_name = {lt.name: lt for lt in compute_lifetimes(kernel)}
    inserts: dict[int, list[AliasFragment]] = {}
    storage_decls: list[str] = []
    kept: set[str] = set()
    dropped: set[str] = set()
    for slot in alias_map.slots:
        if len(slot.tenants) == 1:
            kept.add(slot.name)
            continue
        storage = _storage_name(slot.name)
        storage_decls.append(lds_decl(storage, (slot.size_floats,)))
        dropped.update(slot.tenants)
        prev_death = -1
        for i, tenant in enumerate(slot.tenants):
            lt = by_name[tenant]
            if i == 0:
                at, has_barrier = -1, True  # fresh storage: nothing to wait for
            else:
                seam = [j for j in range(prev_death + 1, lt.birth) if _is_barrier(kernel.fragments[j])]
                if seam:
                    at, has_barrier = seam[-1], True
                else:
                    at, has_barrier = lt.birth - 1, False
            inserts.setdefault(at, []).append(
                AliasFragment(
                    old_name=storage,
                    new_name=tenant,
                    new_shape=lt.shape,
                    preceded_by_barrier=has_barrier,
                )
            )
            prev_death = lt.death
    fragments: list = list(inserts.get(-1, ()))
    for i, frag in enumerate(kernel.fragments):
        fragments.append(frag)
        fragments.extend(inserts.get(i, ()))
    decls: list[str] = []
    for decl in kernel.ctx.threadgroup_decls:
        name = _decl_name(decl)
        if name in kept:
            decls.append(decl)
        elif name not in dropped:
            raise ValueError(
                f"apply_alias_map: LDS declaration {decl!r} declares name {name!r} which is "
                "not present in any AliasSlot. This means lifetime analysis missed the LDS object."
            )
    decls.extend(storage_decls)
    ctx = dataclasses.replace(kernel.ctx, threadgroup_decls=tuple(decls))
    return Kernel(fragments=tuple(fragments), ctx=ctx)


def apply_group_alias_map(group: KernelGroup, alias_map: AliasMap) -> KernelGroup:
    return dataclasses.replace(group, kernel=apply_alias_map(group.kernel, alias_map))


def alias_group(group: KernelGroup) -> KernelGroup:
    """Lifetimes -> alias plan -> rewritten kernel (the pipeline seam)."""
    return apply_group_alias_map(group, compute_alias_map(compute_lifetimes(group.kernel)))


__all__ = [
    "AliasMap",
    "AliasSlot",
    "FusionBudget",
    "TGMEM_CAP_BYTES",
    "TgmemLifetime",
    "TgmemOverflowError",
    "alias_group",
    "apply_alias_map",
    "apply_group_alias_map",
    "compute_alias_map",
    "compute_budget",
    "compute_group_alias_map",
    "compute_group_budget",
    "compute_group_lifetimes",
    "compute_lifetimes",
]
