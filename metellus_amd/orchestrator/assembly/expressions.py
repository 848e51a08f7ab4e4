"""Chain expression helpers for the assembly templates (reference:
src/orchestrator/assembly/expressions.py:1-205).  The chain compiler itself
lives in ``compute.elementwise.chain``; this module keeps the reference's
closure-style entry points on top of it."""

from __future__ import annotations

from metellus_amd.compute.elementwise.chain import (  # noqa: F401
    ChainCode,
    External,
    scalar_literal,
    substitute,
    wrap_bool,
)
from metellus_amd.orchestrator.assembly.extras import Extras
from metellus_amd.orchestrator.ir import ElementwiseOp


def chain_value_transform(chain, *, row_var, col_var, extras: Extras, base_slot: int, name: str = "chain"):
    """Reference-compatible closure ``raw -> expression`` (reference:
    src/orchestrator/assembly/expressions.py:117-170) built on ``ChainCode``.
    Returns the closure; the helper source is available as ``.helper``."""
    primary = chain[0].operands[0]
    code = ChainCode(tuple(chain), (primary.name,), name)
    code.register_extras(extras, base_slot)

    def transform(raw: str) -> str:
        return code.scalar_call([raw], row_var, col_var)

    transform.helper = code.helper()  # type: ignore[attr-defined]
    transform.code = code  # type: ignore[attr-defined]
    return transform


def build_reduction_epilogue_transform(chain: tuple[ElementwiseOp, ...], name: str = "epilogue"):
    """Closure ``v -> expression`` for a reduction epilogue (unary or
    Scalar-binary ops only)."""
    primary = chain[0].operands[0]
    code = ChainCode(tuple(chain), (primary.name,), name)
    if code.externals:
        raise ValueError("reduction epilogue chains may only use Scalar secondary operands")

    def transform(v: str) -> str:
        return code.call([v], [])

    transform.helper = code.helper()  # type: ignore[attr-defined]
    transform.code = code  # type: ignore[attr-defined]
    return transform
