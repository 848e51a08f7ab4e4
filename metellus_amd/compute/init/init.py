"""Buffer initialisation fragments: fill, arange, copy (reference:
src/compute/init/init.py:15-80, exercised by the reference's
tests/bench_init.py).

Same contract as the reference: one element per lane over a one-dimensional
grid of ``tg_x``-lane workgroups, element ``blockIdx.x * tg_x + lane`` while
it is below ``count_dim``.  The lane index comes from the launch itself
(``threadIdx``), so the fragments need no preamble; each renders inside its
own scope.  Consecutive lanes touch consecutive floats, so every wave64
store covers 256 contiguous bytes.  Values are embedded as float literals,
and non-finite values are rejected as in the reference.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess
from metellus_amd.memory.memory import flat_tid


def _float_literal(value: float) -> str:
    if not math.isfinite(float(value)):
        raise ValueError(f"Cannot embed non-finite float as a HIP literal: {value!r}")
    return f"{float(value)!r}f"


def _element_loop(ctx: CodegenContext, count_dim: str, body: str) -> str:
    return "\n".join(
        [
            "{",
            f"    const unsigned gid = blockIdx.x * {ctx.num_threads}u + {flat_tid(ctx)};",
            f"    if (gid < {count_dim}) {{",
            f"        {body}",
            "    }",
            "}",
        ]
    )


@dataclass(frozen=True)
class FillFragment:
    out_name: str
    count_dim: str
    value: float = 0.0
    name: str = "fill"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        return _element_loop(ctx, self.count_dim, f"{self.out_name}[gid] = {_float_literal(self.value)};")

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class ArangeFragment:
    """``out[i] = start + step * float(i)`` (one rounding for the product and
    one for the sum; fused multiply-add is off in every kernel)."""

    out_name: str
    count_dim: str
    start: float = 0.0
    step: float = 1.0
    name: str = "arange"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        expr = f"{_float_literal(self.start)} + {_float_literal(self.step)} * (float)gid"
        return _element_loop(ctx, self.count_dim, f"{self.out_name}[gid] = {expr};")

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class CopyFragment:
    out_name: str
    in_name: str
    count_dim: str
    name: str = "copy"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        return _element_loop(ctx, self.count_dim, f"{self.out_name}[gid] = {self.in_name}[gid];")

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()
