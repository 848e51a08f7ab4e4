"""Register-resident elementwise kernel body for gfx950.

The reference stages every operand through 16x16 threadgroup tiles
(reference: src/orchestrator/assembly/elementwise.py:17-128).  On CDNA4 the
chain is HBM-bound and LDS staging only adds latency, so here each lane
loads its operands straight into registers with 128-bit loads, applies the
fused chain (a ``ChainCode`` helper) per element and writes 128-bit stores.
No LDS is used (the kernel's LDS budget is 0).

Two layouts:

* ``flat`` -- every tensor operand is dense with the primary's shape (or a
  SCALAR broadcast), so the tensor is walked as one contiguous array of
  E = M*N floats.  A workgroup of NT lanes covers ``NT*4*U`` floats: lane t
  handles the float4 at ``base + u*NT*4 + 4t`` for u < U (all loads are
  issued before any arithmetic).  The last partial vector is done element
  by element.
* ``tiled`` -- general strides and ROW/COL broadcasts.  A wave covers
  ``64/LPR`` rows per step with ``LPR`` lanes per row, each lane ``VEC``
  consecutive columns; a workgroup (NWAVES waves) covers ``TM x TN`` with
  ``TM = NWAVES * (64/LPR) * RPW`` rows.  ``VEC`` is 4 when N % 4 == 0 (each
  operand then uses a 128-bit load if its own strides allow, else 4 scalar
  loads), else 1.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from metellus_amd.compute.elementwise.elementwise import BroadcastSpec
from metellus_amd.compute.fragments import CodegenContext, TgmemAccess
from metellus_amd.compute.elementwise.chain import ChainCode, External, param_name
from metellus_amd.orchestrator.ir import Tensor

NWAVES = 4
NT = 64 * NWAVES

# Streaming policy, chosen by measurement on MI355X with the Infinity Cache
# flushed (C2 chain 4096^2, C3 chains 8192^2): nontemporal 128-bit loads;
# 128-bit stores at device scope (sc1), which on gfx950 write through the
# XCD's L2 instead of leaving dirty lines there (same-process A/B: C2 53.57 ->
# 51.67 us, C3 chains, C4 sigmoid and C5 e chains +2.7-3.5 %; nontemporal
# stores were 4 % slower than ordinary ones); flat: 1024 lanes x 1 float4 per
# lane (the 256-1024 lane, 1-4 float4 variants all land within 3 %); tiled:
# 8 elements per lane.
FLAT_THREADS = 1024
FLAT_UNROLL = 1
TILED_ELEMS = 8  # elements per lane in the tiled layout
NT_LOAD = True
NT_STORE = False
WT_STORE = True


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def _next_pow2(x: int) -> int:
    p = 1
    while p < x:
        p *= 2
    return p


@dataclass(frozen=True)
class StreamLayout:
    kind: str  # "flat" | "tiled"
    vec: int = 4
    unroll: int = 4  # flat: float4 per lane; tiled: rows per lane (RPW)
    lpr: int = 64  # tiled: lanes per row
    threads: int = NT  # lanes per workgroup (flat layout)
    nt_load: bool = NT_LOAD  # nontemporal (streaming) loads
    nt_store: bool = NT_STORE  # nontemporal stores
    wt_store: bool = WT_STORE  # device-scope stores (write through L2); wins over nt_store

    def tile(self) -> tuple[int, int]:
        """(TM, TN) of one workgroup for the tiled layout."""
        return NWAVES * (64 // self.lpr) * self.unroll, self.lpr * self.vec


def _dense_like(t: Tensor, shape: tuple[int, ...]) -> bool:
    return t.shape == shape and t.is_contiguous() and (len(shape) < 2 or t.row_stride == shape[1])


def choose_layout(primary: Tensor, externals: list[External], M: int, N: int) -> StreamLayout:
    flat = _dense_like(primary, primary.shape) and all(
        e.broadcast is BroadcastSpec.SCALAR or (e.broadcast is BroadcastSpec.NONE and _dense_like(e.tensor, primary.shape))
        for e in externals
    )
    if flat:
        assert FLAT_THREADS % 64 == 0 and FLAT_THREADS <= 1024
        return StreamLayout(
            "flat", vec=4, unroll=FLAT_UNROLL, threads=FLAT_THREADS, nt_load=NT_LOAD, nt_store=NT_STORE,
            wt_store=WT_STORE,
        )
    vec = 4 if N % 4 == 0 else 1
    lpr = min(64, _next_pow2(_ceil_div(N, vec)))
    rows_per_step = NWAVES * (64 // lpr)
    rpw = max(1, min(max(1, TILED_ELEMS // vec), _ceil_div(M, rows_per_step)))
    return StreamLayout("tiled", vec=vec, unroll=rpw, lpr=lpr, nt_load=NT_LOAD, nt_store=NT_STORE, wt_store=WT_STORE)


def grid_for_layout(layout: StreamLayout, M: int, N: int) -> tuple[int, int, int]:
    if layout.kind == "flat":
        return (_ceil_div(M * N, layout.threads * 4 * layout.unroll), 1, 1)
    tm, tn = layout.tile()
    return (_ceil_div(N, tn), _ceil_div(M, tm), 1)


def _vector_ok(t: Tensor, bc: BroadcastSpec) -> bool:
    """Can a float4 along columns be loaded with one 128-bit access?"""
    if bc is BroadcastSpec.ROW:
        cs = t.col_stride if len(t.shape) == 2 else t.row_stride
        return cs == 1
    if bc is BroadcastSpec.NONE:
        return len(t.shape) == 2 and t.col_stride == 1 and t.row_stride % 4 == 0
    return False


@dataclass(frozen=True)
class ElementwiseStreamFragment:
    """Loads operands, applies ``code`` and stores to ``out_key``."""

    code: ChainCode = field(compare=False)
    primary: Tensor
    out_key: str
    layout: StreamLayout
    name: str = "elementwise_stream"
    kind: str = "compute"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    # -- operand fetch code ---------------------------------------------------

    def _operands(self) -> list[External]:
        return [External(self.primary, BroadcastSpec.NONE), *self.code.externals]

    def _ld4(self, addr: str) -> str:
        return f"mt_ld4_nt({addr})" if self.layout.nt_load else f"mt_ld4({addr})"

    def _st4(self, addr: str, val: str) -> str:
        if self.layout.wt_store:
            return f"mt_st4_wt({addr}, {val})"
        return f"mt_st4_nt({addr}, {val})" if self.layout.nt_store else f"mt_st4({addr}, {val})"

    def render(self, ctx: CodegenContext) -> str:
        if self.layout.kind == "flat":
            return self._render_flat()
        return self._render_tiled()

    def _render_flat(self) -> str:
        U = self.layout.unroll
        T = self.layout.threads
        out = param_name(self.out_key)
        ops = self._operands()
        lines = [
            "const size_t E = (size_t)M * (size_t)N;",
            f"const size_t base = (size_t)blockIdx.x * {T * 4 * U}u + (size_t)threadIdx.x * 4u;",
        ]
        regs = []
        for k, e in enumerate(ops):
            p = param_name(e.tensor.buffer_key)
            if e.broadcast is BroadcastSpec.SCALAR:
                lines.append(f"const float r{k} = {p}[0];")
                regs.append(("scalar", f"r{k}", p))
            else:
                lines.append(f"mt_f32x4 r{k}[{U}];")
                regs.append(("vec", f"r{k}", p))
        lines.append("#pragma unroll")
        lines.append(f"for (int u = 0; u < {U}; ++u) {{")
        lines.append(f"    const size_t idx = base + (size_t)u * {T * 4}u;")
        lines.append("    if (idx + 4u <= E) {")
        for kind, r, p in regs:
            if kind == "vec":
                lines.append(f"        {r}[u] = {self._ld4(f'{p} + idx')};")
        lines.append("    }")
        lines.append("}")
        lines.append("#pragma unroll")
        lines.append(f"for (int u = 0; u < {U}; ++u) {{")
        lines.append(f"    const size_t idx = base + (size_t)u * {T * 4}u;")
        lines.append("    if (idx + 4u <= E) {")
        lines.append("        mt_f32x4 o;")
        for j in range(4):
            vals = [f"{r}[u][{j}]" if kind == "vec" else r for kind, r, _ in regs]
            lines.append(f"        o[{j}] = {self.code.call(vals[:1], vals[1:])};")
        lines.append(f"        {self._st4(f'{out} + idx', 'o')};")
        lines.append("    } else {")
        lines.append("        for (size_t i = idx; i < E; ++i) {")
        vals = [f"{p}[i]" if kind == "vec" else r for kind, r, p in regs]
        lines.append(f"            {out}[i] = {self.code.call(vals[:1], vals[1:])};")
        lines.append("        }")
        lines.append("    }")
        lines.append("}")
        return "\n".join(lines)

    def _render_tiled(self) -> str:
        lay = self.layout
        tm, tn = lay.tile()
        rps = 64 // lay.lpr
        step = NWAVES * rps
        V = lay.vec
        RPW = lay.unroll
        out = param_name(self.out_key)
        ops = self._operands()
        lines = [
            "const unsigned lane = mt_lane();",
            "const unsigned wave = mt_wave();",
            f"const unsigned col = blockIdx.x * {tn}u + (lane % {lay.lpr}u) * {V}u;",
            f"const unsigned row0 = blockIdx.y * {tm}u + wave * {rps}u + lane / {lay.lpr}u;",
        ]
        # register arrays
        kinds = []
        for k, e in enumerate(ops):
            bc = e.broadcast
            if V == 4 and bc in (BroadcastSpec.NONE, BroadcastSpec.ROW):
                kinds.append("vec")
                lines.append(f"mt_f32x4 r{k}[{RPW}];")
            else:
                kinds.append("scalar")
                lines.append(f"float r{k}[{RPW}];")
        lines.append("#pragma unroll")
        lines.append(f"for (int k = 0; k < {RPW}; ++k) {{")
        lines.append(f"    const unsigned row = row0 + (unsigned)k * {step}u;")
        lines.append("    if (row < M && col < N) {")
        for k, e in enumerate(ops):
            p = param_name(e.tensor.buffer_key)
            if kinds[k] == "vec":
                if _vector_ok(e.tensor, e.broadcast):
                    addr = p + " + " + e.offset("row", "col")
                    lines.append(f"        r{k}[k] = {self._ld4(addr)};")
                else:
                    comps = ", ".join(f"{p}[{e.offset('row', f'col + {j}u')}]" for j in range(4))
                    lines.append(f"        r{k}[k] = mt_f32x4{{{comps}}};")
            else:
                lines.append(f"        r{k}[k] = {p}[{e.offset('row', 'col')}];")
        lines.append("    }")
        lines.append("}")
        lines.append("#pragma unroll")
        lines.append(f"for (int k = 0; k < {RPW}; ++k) {{")
        lines.append(f"    const unsigned row = row0 + (unsigned)k * {step}u;")
        lines.append("    if (row < M && col < N) {")
        if V == 4:
            lines.append("        mt_f32x4 o;")
            for j in range(4):
                vals = [f"r{k}[k][{j}]" if kinds[k] == "vec" else f"r{k}[k]" for k in range(len(ops))]
                lines.append(f"        o[{j}] = {self.code.call(vals[:1], vals[1:])};")
            lines.append(f"        {self._st4(f'{out} + (size_t)row * N + col', 'o')};")
        else:
            vals = [f"r{k}[k]" for k in range(len(ops))]
            lines.append(f"        {out}[(size_t)row * N + col] = {self.code.call(vals[:1], vals[1:])};")
        lines.append("    }")
        lines.append("}")
        return "\n".join(lines)
