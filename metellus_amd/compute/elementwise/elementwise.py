"""Elementwise op table for gfx950 HIP code generation.

Each op is an expression template over the placeholders ``x`` (primary),
``y`` (second operand) and ``cond`` (third operand of ``where``).  The
placeholder convention and the op set follow the reference table
(reference: src/compute/elementwise/elementwise.py:18-58); the right-hand
sides are HIP device expressions for gfx950:

* ``max``/``min`` are ``fmaxf``/``fminf`` (IEEE maxNum/minNum: a NaN operand
  loses to a number), as in the reference's ``fmax``/``fmin``.
* ``tanh`` is the saturating form ``copysign(1 - 2/(1 + exp(2|x|)), x)``
  (reference :27-30) -- it returns +/-1 for large |x| rather than NaN.
* ``sign`` maps NaN to 0 (both comparisons are false), as in the reference.
* comparisons produce a C++ ``bool``; the code generators wrap them into
  ``1.0f``/``0.0f`` (:func:`elementwise_outputs_bool`).

Kernels are compiled with ``-ffp-contract=off`` so ``x * y + z`` in a chain
is two correctly-rounded IEEE operations, exactly what NumPy computes.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from enum import Enum

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess


class BroadcastSpec(str, Enum):
    """How a secondary operand maps onto the (M, N) primary
    (reference: src/compute/elementwise/elementwise.py:8-15).

    NONE = same shape, SCALAR = (1, 1), ROW = (1, N), COL = (M, 1)."""

    NONE = "none"
    SCALAR = "scalar"
    ROW = "row"
    COL = "col"

    def __str__(self) -> str:  # str(BroadcastSpec.ROW) == "row"
        return self.value


UNARY_EXPRESSIONS: dict[str, str] = {
    "negate": "-x",
    "absolute": "fabsf(x)",
    "exp": "expf(x)",
    "log": "logf(x)",
    "sqrt": "sqrtf(x)",
    "recip": "1.0f / x",
    "sin": "sinf(x)",
    "cos": "cosf(x)",
    "tanh": "copysignf(1.0f - 2.0f / (1.0f + expf(2.0f * fabsf(x))), x)",
    "floor": "floorf(x)",
    "ceil": "ceilf(x)",
    "sign": "(x > 0.0f) ? 1.0f : ((x < 0.0f) ? -1.0f : 0.0f)",
}

BINARY_EXPRESSIONS: dict[str, str] = {
    "add": "x + y",
    "subtract": "x - y",
    "mul": "x * y",
    "div": "x / y",
    "max": "fmaxf(x, y)",
    "min": "fminf(x, y)",
    "pow": "powf(x, y)",
    "equal": "x == y",
    "not_equal": "x != y",
    "lt": "x < y",
    "gt": "x > y",
    "ge": "x >= y",
    "le": "x <= y",
}

TERNARY_EXPRESSIONS: dict[str, str] = {
    "where": "cond != 0.0f ? x : y",
}

COMPARISON_OPS = frozenset({"equal", "not_equal", "lt", "gt", "ge", "le"})
BROADCAST_MODES = frozenset(m.value for m in BroadcastSpec)

# Ops whose fp32 result is correctly rounded (or exact), so a GPU result can
# be compared bit-for-bit with NumPy's float32 arithmetic.  Transcendentals
# (exp, log, sin, cos, pow, tanh) come from different libm implementations
# on the two sides and are compared within a tolerance.
IEEE_EXACT_OPS = frozenset(
    {
        "negate", "absolute", "sqrt", "recip", "floor", "ceil", "sign",
        "add", "subtract", "mul", "div", "max", "min",
        "equal", "not_equal", "lt", "gt", "ge", "le", "where",
    }
)


def supported_elementwise_ops() -> tuple[str, ...]:
    return tuple(sorted((*UNARY_EXPRESSIONS, *BINARY_EXPRESSIONS, *TERNARY_EXPRESSIONS)))


def _unknown(op: str) -> ValueError:
    return ValueError(
        f"Unsupported elementwise op {op!r}; expected one of {supported_elementwise_ops()}"
    )


def elementwise_arity(op: str) -> int:
    if op in UNARY_EXPRESSIONS:
        return 1
    if op in BINARY_EXPRESSIONS:
        return 2
    if op in TERNARY_EXPRESSIONS:
        return 3
    raise _unknown(op)


def elementwise_expression(op: str) -> str:
    for table in (UNARY_EXPRESSIONS, BINARY_EXPRESSIONS, TERNARY_EXPRESSIONS):
        if op in table:
            return table[op]
    raise _unknown(op)


def elementwise_outputs_bool(op: str) -> bool:
    elementwise_expression(op)  # validates the name
    return op in COMPARISON_OPS


_PLACEHOLDER = re.compile(r"\b(cond|x|y)\b")


def substitute_placeholders(expr: str, **subs: str) -> str:
    """Replace whole-word ``x``/``y``/``cond`` in an expression template."""
    return _PLACEHOLDER.sub(lambda m: subs.get(m.group(0), m.group(0)), expr)


def elementwise_compute_block(
    op: str,
    output_name: str = "out",
    x_name: str = "x",
    y_name: str = "y",
    cond_name: str = "cond",
) -> str:
    """One assignment statement computing ``op`` into ``output_name``."""
    expr = substitute_placeholders(
        elementwise_expression(op), x=x_name, y=y_name, cond=cond_name
    )
    if elementwise_outputs_bool(op):
        return f"{output_name} = ({expr}) ? 1.0f : 0.0f;"
    return f"{output_name} = {expr};"


# ---------------------------------------------------------------------------
# Stand-alone single-op tile fragment (reference bench-only fragment,
# src/compute/elementwise/elementwise.py:186-277).  Operates on LDS tiles.
# ---------------------------------------------------------------------------


def _tile_ref(tile: str, mode: str, row: str, col: str) -> str:
    if mode == "none":
        return f"{tile}[{row}][{col}]"
    if mode == "scalar":
        return f"{tile}[0][0]"
    if mode == "row":
        return f"{tile}[0][{col}]"
    if mode == "col":
        return f"{tile}[{row}][0]"
    raise ValueError(
        f"Unsupported broadcast mode {mode!r}; expected one of {sorted(BROADCAST_MODES)}"
    )


def _bc_shape(mode: str, shape: tuple[int, int]) -> tuple[int, int]:
    rows, cols = shape
    return {"scalar": (1, 1), "row": (1, cols), "col": (rows, 1)}.get(mode, shape)


def elementwise_threadgroup_section(
    op: str,
    output_tile: str,
    x_tile: str,
    tile_shape: tuple[int, int],
    num_threads: int,
    y_tile: str | None = None,
    cond_tile: str | None = None,
    y_broadcast: str = "none",
    cond_broadcast: str = "none",
) -> str:
    """A strided loop applying ``op`` over an LDS tile (one element per lane
    per iteration).  Used by the bench-only single-op fragment."""
    rows, cols = tile_shape
    arity = elementwise_arity(op)
    if arity >= 2 and y_tile is None:
        raise ValueError(f"{op!r} requires y_tile")
    if arity == 3 and cond_tile is None:
        raise ValueError(f"{op!r} requires cond_tile")
    for label, mode in (("y_broadcast", y_broadcast), ("cond_broadcast", cond_broadcast)):
        if mode not in BROADCAST_MODES:
            raise ValueError(
                f"Unsupported {label} {mode!r}; expected one of {sorted(BROADCAST_MODES)}"
            )
    lines = [
        f"for (unsigned idx = flat_tid; idx < {rows * cols}u; idx += {num_threads}u) {{",
        f"    const unsigned tile_row = idx / {cols}u;",
        f"    const unsigned tile_col = idx % {cols}u;",
        f"    const float x = {x_tile}[tile_row][tile_col];",
    ]
    if arity >= 2:
        lines.append(f"    const float y = {_tile_ref(y_tile, y_broadcast, 'tile_row', 'tile_col')};")
    if arity == 3:
        lines.append(
            f"    const float cond = {_tile_ref(cond_tile, cond_broadcast, 'tile_row', 'tile_col')};"
        )
    lines.append("    " + elementwise_compute_block(op, output_name=f"{output_tile}[tile_row][tile_col]"))
    lines.append("}")
    return "\n".join(lines)


@dataclass(frozen=True)
class ElementwiseComputeFragment:
    """Single elementwise op over LDS tiles (bench-only in the reference)."""

    op: str
    output_tile: str
    x_tile: str
    tile_shape: tuple[int, int]
    num_threads: int
    y_tile: str | None = None
    cond_tile: str | None = None
    y_broadcast: str = "none"
    cond_broadcast: str = "none"
    name: str = "elementwise_compute"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        return elementwise_threadgroup_section(
            op=self.op,
            output_tile=self.output_tile,
            x_tile=self.x_tile,
            tile_shape=self.tile_shape,
            num_threads=self.num_threads,
            y_tile=self.y_tile,
            cond_tile=self.cond_tile,
            y_broadcast=self.y_broadcast,
            cond_broadcast=self.cond_broadcast,
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        shape = self.tile_shape
        out = [TgmemAccess(self.x_tile, "read", shape[0] * shape[1], shape)]
        arity = elementwise_arity(self.op)
        for present, tile, mode in (
            (arity >= 2, self.y_tile, self.y_broadcast),
            (arity == 3, self.cond_tile, self.cond_broadcast),
        ):
            if present and tile is not None:
                s = _bc_shape(mode, shape)
                out.append(TgmemAccess(tile, "read", s[0] * s[1], s))
        out.append(TgmemAccess(self.output_tile, "write", shape[0] * shape[1], shape))
        return tuple(out)
