"""Last-axis reduction fragments for gfx950 (sum / max / min / product).

Replaces the reference's one-threadgroup-per-row simdgroup reduction
(reference: src/compute/reduction/reduction.py:23-205) with a wave64 design:

* ``W`` waves cooperate on a row (``T = 64*W`` lanes) and a 256-lane
  workgroup holds ``R = 4/W`` rows.  W = 1 (one wave per row, no LDS) when
  there are enough rows to fill the GPU; W = 2 or 4 for few, long rows.
* Each lane walks its row in chunks.  Vector path (unit column stride,
  K % 4 == 0, row stride % 4 == 0): lane t reads float4 chunks
  q = t, t+T, t+2T, ... (elements 4q..4q+3) into four accumulators a0..a3
  (a_j sees element 4q+j), then its value is (a0 op a1) op (a2 op a3).
  Scalar path: lane t reads elements t, t+T, ... into a0; its value is a0.
  Up to U chunks are loaded before they are combined, in chunk order.
* The 64 lane values of a wave are combined by the butterfly
  ``v = v op shfl_xor(v, off)`` for off = 32, 16, 8, 4, 2, 1.
* With W > 1 each wave's result goes to LDS ``scratch``; the row's first
  wave folds them left to right: ((w0 op w1) op w2) op w3.
* The optional epilogue is applied to the final value, which lane 0 stores.

This order is fixed and documented so the CPU oracle
(``oracle/ir_eval.py: ordered_row_reduce``) replays it exactly: sums and
products are then bit-identical to the oracle's, not merely close.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess

REDUCTION_OPS = ("sum", "max", "min", "product")

ValueTransform = Callable[[str], str]

# Measured on MI355X with the caches flushed by a read pass before each
# launch: nontemporal loads take an 8192^2 row reduction from ~48 us to
# ~42.5 us (6.3 TB/s) and the 32-head 2048^2 attention reductions from
# ~89 us to ~81 us (6.6 TB/s); unroll 4..32 and 1..4 waves per row move
# either by less than run-to-run noise.
UNROLL = 16  # float4 chunks (or elements) in flight per lane
NT_LOAD = True  # nontemporal (streaming) row loads


def _identity(op: str) -> str:
    return {"sum": "0.0f", "product": "1.0f", "max": "(-INFINITY)", "min": "INFINITY"}[op]


def _combine(op: str, a: str, b: str) -> str:
    if op == "sum":
        return f"{a} + {b}"
    if op == "product":
        return f"{a} * {b}"
    if op == "max":
        return f"fmaxf({a}, {b})"
    if op == "min":
        return f"fminf({a}, {b})"
    raise ValueError(f"unsupported reduction op: {op}")


def _mult4(v: str) -> bool:
    try:
        return int(v) % 4 == 0
    except (TypeError, ValueError):
        return False


def _uint(v: str) -> str:
    """An unsigned operand: integer literals get the ``u`` suffix, anything
    else (a dim name or expression) is parenthesised."""
    try:
        return f"{int(v)}u"
    except (TypeError, ValueError):
        return f"({v})"


def _check_op(op: str) -> None:
    if op not in REDUCTION_OPS:
        raise ValueError(f"unsupported reduction op: {op}")


def scratch_floats(waves_per_row: int, rows_per_group: int) -> int:
    return waves_per_row * rows_per_group if waves_per_row > 1 else 0


@dataclass(frozen=True)
class LastAxisReductionSetupFragment:
    """Declares ``lane``, ``wave``, ``row`` (this lane's row), ``t`` (lane
    index within the row's T lanes) and ``row_ok``."""

    rows_dim: str
    name: str
    waves_per_row: int | None = None
    rows_per_group: int = 1
    kind: str = "setup"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    def render(self, ctx: CodegenContext) -> str:
        W = self.waves_per_row or max(1, ctx.tg_x // 64)
        R = self.rows_per_group
        return "\n".join(
            [
                "const unsigned lane = mt_lane();",
                "const unsigned wave = mt_wave();",
                f"const unsigned row = blockIdx.x * {R}u + wave / {W}u;",
                f"const unsigned t = (wave % {W}u) * 64u + lane;",
                f"const bool row_ok = row < {self.rows_dim};",
            ]
        )


@dataclass(frozen=True)
class LastAxisReductionComputeFragment:
    """Per-row reduction of ``input_name[row*row_stride + idx*col_stride]``
    over ``idx < reduce_dim``; ``value_transform`` wraps each element (it may
    use ``row`` and ``idx``).  Leaves the lane's wave-reduced value in ``r``
    (valid in the row's first wave)."""

    op: str
    input_name: str
    scratch_name: str
    reduce_dim: str
    row_stride: str
    name: str
    tg_x: int
    col_stride: str = "1"
    value_transform: ValueTransform | None = None
    waves_per_row: int | None = None
    rows_per_group: int = 1
    vectorized: bool | None = None
    unroll: int = UNROLL
    nt_load: bool = NT_LOAD
    kind: str = "compute"

    @property
    def W(self) -> int:
        return self.waves_per_row or max(1, self.tg_x // 64)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        n = scratch_floats(self.W, self.rows_per_group)
        if n == 0:
            return ()
        return (TgmemAccess(self.scratch_name, "readwrite", n, (n,)),)

    def _vec(self) -> bool:
        """128-bit loads need contiguous rows whose length and stride are
        known multiples of 4 (the vector loop covers ``reduce_dim / 4``
        quads and nothing else); symbolic sizes take the per-element loop."""
        if self.vectorized is not None:
            return self.vectorized
        return self.col_stride == "1" and _mult4(self.reduce_dim) and _mult4(self.row_stride)

    def render(self, ctx: CodegenContext) -> str:
        _check_op(self.op)
        W, T = self.W, 64 * self.W
        U = self.unroll
        ld4 = "mt_ld4_nt" if self.nt_load else "mt_ld4"
        ident = _identity(self.op)
        tf = self.value_transform or (lambda raw: raw)
        src = f"{self.input_name} + (size_t)row * {_uint(self.row_stride)}"
        L = [f"float a0 = {ident}, a1 = {ident}, a2 = {ident}, a3 = {ident};", "if (row_ok) {",
             f"    const float* __restrict__ src = {src};"]
        if self._vec():
            L += [
                f"    const unsigned nq = {self.reduce_dim} / 4u;",
                "    unsigned q = t;",
                f"    for (; q + {(U - 1) * T}u < nq; q += {U * T}u) {{",
                f"        mt_f32x4 x[{U}];",
                "#pragma unroll",
                f"        for (int u = 0; u < {U}; ++u) x[u] = {ld4}(src + 4u * (q + (unsigned)u * {T}u));",
                "#pragma unroll",
                f"        for (int u = 0; u < {U}; ++u) {{",
            ]
            for j in range(4):
                L += [
                    f"            {{ const unsigned idx = 4u * (q + (unsigned)u * {T}u) + {j}u; (void)idx;",
                    f"              a{j} = {_combine(self.op, f'a{j}', tf(f'x[u][{j}]'))}; }}",
                ]
            L += [
                "        }",
                "    }",
                f"    for (; q < nq; q += {T}u) {{",
                f"        const mt_f32x4 xv = {ld4}(src + 4u * q);",
            ]
            for j in range(4):
                L += [
                    f"        {{ const unsigned idx = 4u * q + {j}u; (void)idx;",
                    f"          a{j} = {_combine(self.op, f'a{j}', tf(f'xv[{j}]'))}; }}",
                ]
            L += ["    }"]
        else:
            cs = self.col_stride
            load = "src[idx]" if cs == "1" else f"src[(size_t)idx * {_uint(cs)}]"
            L += [
                "    unsigned e = t;",
                f"    for (; e + {(U - 1) * T}u < {self.reduce_dim}; e += {U * T}u) {{",
                f"        float x[{U}];",
                "#pragma unroll",
                f"        for (int u = 0; u < {U}; ++u) {{ const unsigned idx = e + (unsigned)u * {T}u; x[u] = {load}; }}",
                "#pragma unroll",
                f"        for (int u = 0; u < {U}; ++u) {{",
                f"            const unsigned idx = e + (unsigned)u * {T}u; (void)idx;",
                f"            a0 = {_combine(self.op, 'a0', tf('x[u]'))};",
                "        }",
                "    }",
                f"    for (; e < {self.reduce_dim}; e += {T}u) {{",
                f"        const unsigned idx = e; const float xv = {load};",
                f"        a0 = {_combine(self.op, 'a0', tf('xv'))};",
                "    }",
            ]
        L += ["}"]
        if self._vec():
            lo = "(" + _combine(self.op, "a0", "a1") + ")"
            hi = "(" + _combine(self.op, "a2", "a3") + ")"
            L.append(f"float r = {_combine(self.op, lo, hi)};")
        else:
            L.append("float r = a0;")
        L.append(f"r = mt_wave_{self.op}(r);")
        if W > 1:
            sc = self.scratch_name
            L += [
                f"if (lane == 0u) {sc}[wave] = r;",
                "__syncthreads();",
                f"if (wave % {W}u == 0u) {{",
                f"    r = {sc}[wave];",
            ]
            for w in range(1, W):
                L.append(f"    r = {_combine(self.op, 'r', f'{sc}[wave + {w}u]')};")
            L.append("}")
        return "\n".join(L)


@dataclass(frozen=True)
class StoreReductionResultFragment:
    """Lane 0 of the row's first wave stores ``r`` (optionally transformed)."""

    output_name: str
    scratch_name: str
    name: str
    tg_x: int
    value_transform: ValueTransform | None = None
    setup: tuple[str, ...] = ()
    waves_per_row: int | None = None
    kind: str = "store"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    def render(self, ctx: CodegenContext) -> str:
        W = self.waves_per_row or max(1, self.tg_x // 64)
        lines = ["float v = r;", *self.setup]
        if self.value_transform is not None:
            lines.append(f"v = {self.value_transform('v')};")
        lines.append(f"{self.output_name}[row] = v;")
        body = "\n    ".join(lines)
        return f"if (row_ok && lane == 0u && wave % {W}u == 0u) {{\n    {body}\n}}"
