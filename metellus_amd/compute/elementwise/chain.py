"""Compile fused elementwise chains into HIP device code (compute layer).

A chain is a tuple of ``ElementwiseOp``s where each op's primary is the
previous op's output (the first op's primary is the chain *seed*).  Secondary
operands are Scalars (inlined literals), values computed earlier in the
chain (registers), or *external* tensors read from global memory.

``ChainCode`` turns a chain into one ``__device__`` helper

    float <name>(float x, float e0, float e1, ...) { float v0 = ...; ...; return vN; }

whose parameters are the seed value and one value per external operand; the
calling template decides how the externals are fetched (128-bit vectors in
streaming kernels, scalar loads in matmul prologues, ...).  Per-op expression
text follows the reference's chain emission (reference:
src/compute/elementwise/tiled_chain.py:65-79, src/orchestrator/assembly/
expressions.py:33-170): ``float v{i} = <template with x/y/cond substituted>``,
comparison results wrapped to 1.0f/0.0f.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from metellus_amd.compute.elementwise.elementwise import (
    BroadcastSpec,
    elementwise_arity,
    elementwise_expression,
    elementwise_outputs_bool,
    substitute_placeholders,
)
from metellus_amd.orchestrator.ir import ElementwiseOp, Scalar, Tensor


def param_name(buffer_key: str) -> str:
    """Kernel-parameter identifier for a buffer.  Prefixed so user tensor
    names can never collide with the generated locals (``M``, ``row``...)."""
    if buffer_key.isidentifier() and buffer_key.isascii():
        return f"g_{buffer_key}"
    return "g_x" + buffer_key.encode().hex()


def substitute(expr: str, **subs: str) -> str:
    return substitute_placeholders(expr, **subs)


def wrap_bool(op: str, expr: str) -> str:
    if elementwise_outputs_bool(op):
        return f"(({expr}) ? 1.0f : 0.0f)"
    return expr


def scalar_literal(value: float) -> str:
    """fp32 literal (``f`` suffix); inf/nan become ``INFINITY``/``NAN``."""
    if math.isnan(value):
        return "NAN"
    if math.isinf(value):
        return "INFINITY" if value > 0 else "(-INFINITY)"
    text = repr(float(value))
    return f"{text}f"


@dataclass(frozen=True)
class External:
    """A tensor operand of the chain read from global memory."""

    tensor: Tensor
    broadcast: BroadcastSpec

    @property
    def key(self) -> tuple:
        t = self.tensor
        return (t.buffer_key, t.row_stride, t.col_stride, self.broadcast)

    def offset(self, row: str, col: str) -> str:
        """Element offset of this operand at output position (row, col)."""
        t = self.tensor
        if self.broadcast is BroadcastSpec.SCALAR:
            return "0"
        if self.broadcast is BroadcastSpec.ROW:
            return _term(col, t.col_stride) if len(t.shape) == 2 else _term(col, t.row_stride)
        if self.broadcast is BroadcastSpec.COL:
            return _term(row, t.row_stride)
        if len(t.shape) == 1:
            return _term(row, t.row_stride)
        return _sum(_term(row, t.row_stride), _term(col, t.col_stride))

    def scalar_fetch(self, row: str, col: str) -> str:
        return f"{param_name(self.tensor.buffer_key)}[{self.offset(row, col)}]"


def _term(var: str, stride: int) -> str:
    if stride == 0:
        return "0"
    if stride == 1:
        return f"(size_t)({var})"
    return f"(size_t)({var}) * {stride}u"


def _sum(a: str, b: str) -> str:
    if a == "0":
        return b
    if b == "0":
        return a
    return f"{a} + {b}"


FAST_DIVISION = {"div": "mt_div_fast(x, y)", "recip": "mt_div_fast(1.0f, x)"}
# The same divisions when the divisor is known to be plain (mt_div_plain):
# mt_div_fast's own first path, with no test.
PLAIN_DIVISION = {"div": "(x) * mt_div_rcp(y)", "recip": "mt_div_rcp(x)"}


@dataclass
class ChainCode:
    """Device helper for ``chain`` with ``seeds`` (names bound to the helper's
    leading parameters, in order) already in registers."""

    chain: tuple[ElementwiseOp, ...]
    seeds: tuple[str, ...]
    name: str
    externals: list[External] = field(default_factory=list)
    # Divisions feeding a matmul (operand prologues) use mt_div_fast: within
    # 2 ulp of the IEEE quotient, which the matmul bar (1e-4 sqrt(K)) leaves
    # no trace of.  Epilogues and multi-anchor merges produce the kernel's
    # output and keep IEEE division, so a fused chain rounds exactly like
    # the same chain in its own elementwise kernel.
    fast_div: bool = False

    def __post_init__(self) -> None:
        avail = set(self.seeds)
        seen: dict[tuple, int] = {}
        self._operand_ext: dict[tuple[int, int], int] = {}
        for i, op in enumerate(self.chain):
            for pos in range(1, elementwise_arity(op.op)):
                o = op.operands[pos]
                if isinstance(o, Tensor) and o.name not in avail:
                    bc = op.y_broadcast if pos == 1 else op.cond_broadcast
                    ext = External(o, bc)
                    if ext.key not in seen:
                        seen[ext.key] = len(self.externals)
                        self.externals.append(ext)
                    self._operand_ext[(i, pos)] = seen[ext.key]
            avail.add(op.out.name)

    def register_extras(self, extras, base_slot: int) -> None:
        """Add external operands to the kernel's extra buffers, in the
        reference's first-appearance order."""
        for i, op in enumerate(self.chain):
            for pos in range(1, elementwise_arity(op.op)):
                if (i, pos) in self._operand_ext:
                    extras.add_tensor(op.operands[pos], base_slot)

    @property
    def broadcast_operands_only(self) -> bool:
        """True when every external operand is a row, column or scalar
        broadcast (small, cache-resident reads)."""
        small = (BroadcastSpec.ROW, BroadcastSpec.COL, BroadcastSpec.SCALAR)
        return all(e.broadcast in small for e in self.externals)

    def external_axes(self) -> frozenset[str]:
        """Output coordinates (``"row"``, ``"col"``) the external operands'
        values depend on -- read off the same offsets the gathers emit."""
        axes = set()
        for e in self.externals:
            off = e.offset("mt_r_", "mt_c_")
            if "mt_r_" in off:
                axes.add("row")
            if "mt_c_" in off:
                axes.add("col")
        return frozenset(axes)

    @property
    def arity(self) -> int:
        return len(self.seeds) + len(self.externals)

    def helper(self, plain: bool = False) -> str:
        """The chain as a device function ``name(s..., e...)``.  ``plain``:
        ``name_plain``, its divisions reduced to x * mt_div_rcp(y), exact
        when every divisor is plain (``plain_divisors``)."""
        params = [f"float s{k}" for k in range(len(self.seeds))]
        params += [f"float e{k}" for k in range(len(self.externals))]
        local: dict[str, str] = {name: f"s{k}" for k, name in enumerate(self.seeds)}
        lines = []
        cur = f"s0" if self.seeds else None
        for i, op in enumerate(self.chain):
            head = op.operands[0]
            x = local.get(head.name, cur) if isinstance(head, Tensor) else cur
            subs = {"x": f"({x})"}
            for pos, ph in ((1, "y"), (2, "cond")):
                if pos >= elementwise_arity(op.op):
                    continue
                o = op.operands[pos]
                if isinstance(o, Scalar):
                    subs[ph] = f"({scalar_literal(o.value)})"
                elif (i, pos) in self._operand_ext:
                    subs[ph] = f"(e{self._operand_ext[(i, pos)]})"
                else:
                    subs[ph] = f"({local[o.name]})"
            template = elementwise_expression(op.op)
            if self.fast_div and op.op in FAST_DIVISION:
                template = (PLAIN_DIVISION if plain else FAST_DIVISION)[op.op]
            expr = wrap_bool(op.op, substitute(template, **subs))
            lines.append(f"    const float v{i} = {expr};")
            cur = f"v{i}"
            local[op.out.name] = cur
        body = "\n".join(lines)
        result = cur if cur is not None else "0.0f"
        name = f"{self.name}_plain" if plain else self.name
        return (
            f"__device__ __forceinline__ float {name}({', '.join(params)}) {{\n"
            f"{body}\n    return {result};\n}}"
        )

    def plain_divisors(self) -> list[int] | None:
        """Indices k of the gathered operands e_k that are the divisors of the
        chain's fast divisions, when every such divisor is one (then whether
        they are plain is known from the gathered values alone); None when
        the chain has no fast division or one divides by anything else."""
        if not self.fast_div:
            return None
        ks: list[int] = []
        for i, op in enumerate(self.chain):
            if op.op not in FAST_DIVISION:
                continue
            if op.op == "recip" or (i, 1) not in self._operand_ext:
                return None
            ks.append(self._operand_ext[(i, 1)])
        return sorted(set(ks)) or None

    def helpers(self) -> list[str]:
        """The helper, and its plain form when ``plain_divisors`` applies."""
        return [self.helper(), *([self.helper(plain=True)] if self.plain_divisors() else [])]

    def plain_apply_lambda(self) -> str:
        """``apply_lambda`` calling the plain helper."""
        n = len(self.externals)
        args = ", ".join(["raw", *(f"e.v[{k}]" for k in range(n))])
        return f"[=](float raw, const mt_vals<{n}>& e) -> float {{ return {self.name}_plain({args}); }}"

    def plain_predicate_lambda(self) -> str:
        """``[=](const mt_vals<E>& e) -> bool``: every divisor plain."""
        n = len(self.externals)
        test = " && ".join(f"mt_div_plain(e.v[{k}])" for k in self.plain_divisors())
        return f"[=](const mt_vals<{n}>& e) -> bool {{ return {test}; }}"

    def call(self, seed_values: list[str], ext_values: list[str]) -> str:
        return f"{self.name}({', '.join([*seed_values, *ext_values])})"

    def scalar_call(self, seed_values: list[str], row: str, col: str) -> str:
        """Call with every external fetched by a scalar load at (row, col)."""
        return self.call(seed_values, [e.scalar_fetch(row, col) for e in self.externals])

    def gather_lambda(self, row: str = "global_row", col: str = "global_col") -> str:
        """``[=](unsigned row, unsigned col) -> mt_vals<E>``: this element's
        external operands, loaded with the tile (gather / apply loaders)."""
        n = len(self.externals)
        loads = " ".join(f"o.v[{k}] = {e.scalar_fetch(row, col)};" for k, e in enumerate(self.externals))
        return f"[=](unsigned {row}, unsigned {col}) -> mt_vals<{n}> {{ mt_vals<{n}> o; {loads} return o; }}"

    def apply_lambda(self) -> str:
        """``[=](float raw, const mt_vals<E>& e) -> float``: the chain over a
        loaded element and its gathered operands."""
        n = len(self.externals)
        return (
            f"[=](float raw, const mt_vals<{n}>& e) -> float "
            f"{{ return {self.call(['raw'], [f'e.v[{k}]' for k in range(n)])}; }}"
        )

    def lambda_transform(self, row: str = "global_row", col: str = "global_col") -> str:
        """``[=](float raw, unsigned row, unsigned col) -> float`` applying the
        chain to a loaded element (matmul / reduction prologues)."""
        return (
            f"[=](float raw, unsigned {row}, unsigned {col}) -> float "
            f"{{ return {self.scalar_call(['raw'], row, col)}; }}"
        )
