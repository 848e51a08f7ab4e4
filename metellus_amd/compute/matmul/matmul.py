"""Matmul fragments for gfx950: fp32 MFMA mainloop with register epilogues.

Same fragment roles as the reference (reference:
src/compute/matmul/matmul.py:12-369) -- tile mapping, thread index, setup,
mainloop(loads, barrier, compute, barrier), stores -- re-designed for CDNA4:

* accumulators are ``mt_f32x16 acc[WM][WN]`` (32x32 MFMA blocks) per wave;
* ``MatmulMainloopFragment`` renders its loads/compute as a software
  pipeline over double-buffered LDS: the next k-chunk's global loads are in
  flight while the current chunk's MFMAs run, with one barrier per chunk;
* epilogues run on the accumulator registers -- the MFMA output layout is
  fixed (``mt_acc_row``), so every register knows its (row, col) and any
  elementwise chain (scalar, row/col/full-tile operands) applies in place,
  then results go straight to global memory.  No C tile in LDS.
"""

from __future__ import annotations

import textwrap
from dataclasses import dataclass, field
from typing import Any

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess
from metellus_amd.compute.matmul.config import TileConfig

KernelFragment = Any


@dataclass(frozen=True)
class MatmulConfig:
    tile: TileConfig
    aligned: bool
    M_dim_var: str
    K_dim_var: str
    N_dim_var: str
    a_buffer_name: str
    b_buffer_name: str
    c_buffer_name: str
    a_tile_name: str
    b_tile_name: str
    c_tile_name: str = "C_tile"
    c_col_stride: str = "1"

    def validate(self) -> None:
        self.tile.validate()


@dataclass(frozen=True)
class PersistentTiles:
    """Persistent tile loop: a grid of (P, 1, batch) workgroups, workgroup x
    taking output tiles x, x + P, x + 2P, ... (row-major over the
    ``ceil(M / tile_M) x ceil(N / tile_N)`` tiles).  Used when the tiles
    outnumber the workgroups the GPU holds at once: the next tile's first
    k-chunk is then loaded during the current tile's last one, and the
    current tile's stores drain while the next tile's MFMAs run, instead of
    each workgroup paying its own launch, first load and store phases."""

    tile_M: int
    tile_N: int
    M_dim_var: str = "M"
    N_dim_var: str = "N"


@dataclass(frozen=True)
class MatmulTileMappingFragment:
    """``tg`` = (column tile, row tile) of this workgroup; with ``persistent``
    it opens the tile loop (closed by ``PersistentLoopEndFragment``) and
    defines ``mt_first_tile``, ``mt_has_next``, ``mt_next_m0/n0`` for the
    mainloop's cross-tile prefetch."""

    persistent: PersistentTiles | None = None
    name: str = "tile_mapping"
    kind: str = "setup"

    def render(self, ctx: CodegenContext) -> str:
        p = self.persistent
        if p is None:
            return "const uint3 tg = make_uint3(blockIdx.x, blockIdx.y, blockIdx.z);"
        return "\n".join(
            [
                f"const unsigned mt_tiles_x = ({p.N_dim_var} + {p.tile_N - 1}u) / {p.tile_N}u;",
                f"const unsigned mt_tiles = mt_tiles_x * (({p.M_dim_var} + {p.tile_M - 1}u) / {p.tile_M}u);",
                "unsigned mt_stage = 0u;  // LDS buffer holding the current k-chunk",
                "for (unsigned mt_t = blockIdx.x; mt_t < mt_tiles; mt_t += gridDim.x) {",
                "const bool mt_first_tile = mt_t == blockIdx.x;",
                "const unsigned mt_t_next = mt_t + gridDim.x;",
                "const bool mt_has_next = mt_t_next < mt_tiles;",
                f"const unsigned mt_next_m0 = (mt_t_next / mt_tiles_x) * {p.tile_M}u;",
                f"const unsigned mt_next_n0 = (mt_t_next % mt_tiles_x) * {p.tile_N}u;",
                "const uint3 tg = make_uint3(mt_t % mt_tiles_x, mt_t / mt_tiles_x, blockIdx.z);",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class PersistentLoopEndFragment:
    """Closes the persistent tile loop opened by the tile mapping."""

    name: str = "persistent_loop_end"
    kind: str = "setup"

    def render(self, ctx: CodegenContext) -> str:
        return "}  // persistent tile loop"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class ThreadIndexFragment:
    tile: TileConfig
    name: str = "thread_index"
    kind: str = "setup"

    def render(self, ctx: CodegenContext) -> str:
        t = self.tile
        return "\n".join(
            [
                "const unsigned lane = mt_lane();",
                "const unsigned wave = mt_wave();",
                f"const unsigned wave_m0 = (wave / {t.sg_N}u) * {t.wave_M}u;",
                f"const unsigned wave_n0 = (wave % {t.sg_N}u) * {t.wave_N}u;",
                f"const unsigned tile_m0 = tg.y * {t.tile_M}u;",
                f"const unsigned tile_n0 = tg.x * {t.tile_N}u;",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class MatmulSetupFragment:
    """Zeroed accumulators ``acc{suffix}[WM][WN]``."""

    config: MatmulConfig
    accumulator_suffix: str = ""
    emit_thread_coords: bool = True
    name: str = "matmul_setup"
    kind: str = "setup"

    def render(self, ctx: CodegenContext) -> str:
        t = self.config.tile
        a = f"acc{self.accumulator_suffix}"
        return "\n".join(
            [
                f"mt_f32x16 {a}[{t.WM}][{t.WN}];",
                "#pragma unroll",
                f"for (int i = 0; i < {t.WM}; ++i)",
                "#pragma unroll",
                f"    for (int j = 0; j < {t.WN}; ++j) mt_zero({a}[i][j]);",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class MatmulComputeFragment:
    """MFMAs over the LDS k-chunk in buffer ``stage`` (set by the mainloop)."""

    config: MatmulConfig
    accumulator_suffix: str = ""
    name: str = "matmul_compute"
    kind: str = "compute"

    def render_stage(self, stage: str | None) -> str:
        """MFMAs over LDS buffer ``stage`` of double-buffered tiles, or over
        single-buffered tiles when ``stage`` is None."""
        t = self.config.tile
        at, bt = self.config.a_tile_name, self.config.b_tile_name
        a_ptr = f"&{at}[{stage}][wave_m0][0]" if stage is not None else f"&{at}[wave_m0][0]"
        b_ptr = f"&{bt}[{stage}][0][wave_n0]" if stage is not None else f"&{bt}[0][wave_n0]"
        return (
            f"mt_mfma_tile<{t.WM}, {t.WN}, {t.tile_K}, {t.lda}, {t.ldb}>"
            f"({a_ptr}, {b_ptr}, acc{self.accumulator_suffix}, lane);"
        )

    def render(self, ctx: CodegenContext) -> str:
        return self.render_stage("0" if self.config.tile.stages > 1 else None)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        t = self.config.tile
        a_shape = t.a_tile_shape() if t.stages > 1 else t.a_tile_shape()[1:]
        b_shape = t.b_tile_shape() if t.stages > 1 else t.b_tile_shape()[1:]
        return (
            TgmemAccess(self.config.a_tile_name, "read", _prod(a_shape), a_shape),
            TgmemAccess(self.config.b_tile_name, "read", _prod(b_shape), b_shape),
        )


def _prod(shape) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


@dataclass(frozen=True)
class MatmulMainloopFragment:
    """Pipelined k loop over ``fragments`` = (loads..., barrier, computes...,
    barrier) -- the reference's composition (reference:
    src/orchestrator/assembly/matmul.py:187-197).  Rendered as::

        fetch(0); commit(0); barrier
        for kt: if (next) fetch(kt+1); compute(kt&1); if (next) commit((kt+1)&1); barrier

    With two LDS buffers one barrier per chunk suffices: buffer b is written
    in iteration kt only after every lane passed the barrier that ended
    iteration kt-1, the last reader of b.

    ``persistent`` (inside a persistent tile loop): the buffer index is the
    running ``mt_stage``, flipped after every chunk of every tile; only the
    first tile loads chunk 0 before its loop, and the last iteration of each
    tile loads chunk 0 of the next tile (``mt_next_m0/n0``) into the other
    buffer, so the same one-barrier-per-chunk argument spans tiles."""

    tile_K: int
    fragments: tuple[KernelFragment, ...]
    K_dim_var: str
    persistent: bool = False
    name: str = "matmul_mainloop"
    kind: str = "compute"

    def _loads(self):
        return [f for f in self.fragments if hasattr(f, "render_fetch")]

    def _computes(self):
        return [f for f in self.fragments if isinstance(f, MatmulComputeFragment)]

    def render(self, ctx: CodegenContext) -> str:
        loads, computes = self._loads(), self._computes()
        stages = max((ld.stages for ld in loads), default=1)
        kvar = self.K_dim_var
        tk = self.tile_K
        body: list[str] = [ld.render_decl() for ld in loads]
        if stages == 1:
            body += [
                f"for (unsigned k_chunk = 0; k_chunk < {kvar}; k_chunk += {tk}u) {{",
                *[f"    {ld.render_fetch()}" for ld in loads],
                *[f"    {ld.render_commit('0')}" for ld in loads],
                "    __syncthreads();",
                *[f"    {c.render_stage(None)}" for c in computes],
                "    __syncthreads();",
                "}",
            ]
            return "{\n" + textwrap.indent("\n".join(body), "    ") + "\n}"
        if self.persistent:
            if stages != 2:
                raise ValueError("a persistent tile loop needs double-buffered LDS tiles")
            return self._render_persistent(loads, computes, body)
        body += [
            f"const unsigned n_chunks = ({kvar} + {tk - 1}u) / {tk}u;",
            "{",
            "    const unsigned k_chunk = 0u;",
            *[f"    {ld.render_fetch()}" for ld in loads],
            "}",
            *[ld.render_commit("0") for ld in loads],
            "__syncthreads();",
            "for (unsigned kt = 0; kt < n_chunks; ++kt) {",
            "    const unsigned cur = kt & 1u;",
            "    const bool more = kt + 1u < n_chunks;",
            "    if (more) {",
            f"        const unsigned k_chunk = (kt + 1u) * {tk}u;",
            *[f"        {ld.render_fetch()}" for ld in loads],
            "    }",
            *[f"    {c.render_stage('cur')}" for c in computes],
            "    if (more) {",
            *[f"        {ld.render_commit('cur ^ 1u')}" for ld in loads],
            "    }",
            "    __syncthreads();",
            "}",
        ]
        return "{\n" + textwrap.indent("\n".join(body), "    ") + "\n}"

    def _render_persistent(self, loads, computes, body: list[str]) -> str:
        kvar, tk = self.K_dim_var, self.tile_K
        body += [
            f"const unsigned n_chunks = ({kvar} + {tk - 1}u) / {tk}u;",
            "if (mt_first_tile) {",
            "    const unsigned k_chunk = 0u;",
            *[f"    {ld.render_fetch()}" for ld in loads],
            *[f"    {ld.render_commit('mt_stage')}" for ld in loads],
            "    __syncthreads();",
            "}",
            "for (unsigned kt = 0; kt < n_chunks; ++kt) {",
            "    const unsigned cur = mt_stage;",
            "    const bool more = kt + 1u < n_chunks;",
            "    if (more) {",
            f"        const unsigned k_chunk = (kt + 1u) * {tk}u;",
            *[f"        {ld.render_fetch()}" for ld in loads],
            "    } else if (mt_has_next) {",
            "        const unsigned tile_m0 = mt_next_m0;",
            "        const unsigned tile_n0 = mt_next_n0;",
            "        const unsigned k_chunk = 0u;",
            *[f"        {ld.render_fetch()}" for ld in loads],
            "    }",
            *[f"    {c.render_stage('cur')}" for c in computes],
            "    if (more || mt_has_next) {",
            *[f"        {ld.render_commit('cur ^ 1u')}" for ld in loads],
            "    }",
            "    __syncthreads();",
            "    mt_stage ^= 1u;",
            "}",
        ]
        return "{\n" + textwrap.indent("\n".join(body), "    ") + "\n}"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    @property
    def sub_fragments(self) -> tuple[KernelFragment, ...]:
        return self.fragments


def _epilogue_lines(t: TileConfig, out: str, value: str, check: bool, M: str, N: str) -> str:
    """Loop over every accumulator register: row/col from the MFMA layout,
    ``value`` (an expression over ``i, j, v, row, col``) stored to ``out``."""
    guard = f"if (row < {M} && col < {N}) " if check else ""
    return "\n".join(
        [
            "#pragma unroll",
            f"for (int i = 0; i < {t.WM}; ++i) {{",
            "#pragma unroll",
            f"    for (int j = 0; j < {t.WN}; ++j) {{",
            "        const unsigned col = tile_n0 + wave_n0 + (unsigned)j * 32u + (lane & 31u);",
            "#pragma unroll",
            "        for (int v = 0; v < 16; ++v) {",
            "            const unsigned row = tile_m0 + wave_m0 + (unsigned)i * 32u + mt_acc_row(v, lane);",
            f"            {guard}{out}[(size_t)row * {N} + col] = {value};",
            "        }",
            "    }",
            "}",
        ]
    )


@dataclass(frozen=True)
class MatmulEpilogueStoreFragment:
    """Apply an epilogue to each accumulator value in registers and store it.

    ``value_expr`` is a format string over ``{a}`` (the accumulator value of
    each anchor, in order: ``{a0}``, ``{a1}``), ``row`` and ``col``;
    ``None`` stores the raw accumulator."""

    config: MatmulConfig
    value_expr: str | None = None
    suffixes: tuple[str, ...] = ("",)
    check: bool = False
    name: str = "matmul_epilogue_store"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        vals = {f"a{k}": f"acc{s}[i][j][v]" for k, s in enumerate(self.suffixes)}
        value = self.value_expr.format(**vals) if self.value_expr else vals["a0"]
        cfg = self.config
        return _epilogue_lines(cfg.tile, cfg.c_buffer_name, value, self.check, cfg.M_dim_var, cfg.N_dim_var)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class MatmulAccumToDevFragment:
    """Store raw accumulators to the output (reference name, aligned path)."""

    config: MatmulConfig
    name: str = "matmul_accum_to_dev"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        return MatmulEpilogueStoreFragment(self.config, check=not self.config.aligned).render(ctx)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class MatmulAccumToTgFragment:
    """Accumulators -> the LDS tile ``C_tile[tile_M][tile_N + c_pad]``
    (reference: src/compute/matmul/matmul.py:270-313).  A barrier must follow
    before the tile is read.  The kernels this package assembles keep
    epilogues in registers and never stage C through LDS; this fragment and
    ``MatmulTgToDevFragment`` serve hand-composed kernels."""

    config: MatmulConfig
    accumulator_suffix: str = ""
    emit_tg_coords: bool = True
    name: str = "matmul_accum_to_tg"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        t = self.config.tile
        c = self.config.c_tile_name
        a = f"acc{self.accumulator_suffix}"
        return "\n".join(
            [
                "#pragma unroll",
                f"for (int i = 0; i < {t.WM}; ++i) {{",
                "#pragma unroll",
                f"    for (int j = 0; j < {t.WN}; ++j) {{",
                "#pragma unroll",
                "        for (int v = 0; v < 16; ++v) {",
                f"            {c}[wave_m0 + (unsigned)i * 32u + mt_acc_row(v, lane)]"
                f"[wave_n0 + (unsigned)j * 32u + (lane & 31u)] = {a}[i][j][v];",
                "        }",
                "    }",
                "}",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        t = self.config.tile
        shape = (t.tile_M, t.tile_N + t.c_pad)
        return (TgmemAccess(self.config.c_tile_name, "write", _prod(shape), shape),)


@dataclass(frozen=True)
class MatmulTgToDevFragment:
    """LDS ``C_tile`` -> the output, masked to (M, N) (reference:
    src/compute/matmul/matmul.py:317-352)."""

    config: MatmulConfig
    name: str = "matmul_tg_to_dev"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        from metellus_amd.memory.memory import TgStoreFragment

        t = self.config.tile
        return TgStoreFragment(
            name="store_C_tile",
            src_name=self.config.c_tile_name,
            dst_name=self.config.c_buffer_name,
            dst_row_stride=self.config.N_dim_var,
            row_start="tile_m0",
            col_start="tile_n0",
            tile_shape=(t.tile_M, t.tile_N),
            num_threads=t.num_threads,
            row_limit=self.config.M_dim_var,
            col_limit=self.config.N_dim_var,
            dst_col_stride=self.config.c_col_stride,
        ).render(ctx)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        t = self.config.tile
        shape = (t.tile_M, t.tile_N + t.c_pad)
        return (TgmemAccess(self.config.c_tile_name, "read", _prod(shape), shape),)


@dataclass(frozen=True)
class MatmulRegisterEpilogueFragment:
    """Rewrite accumulators in place with ``value_transform`` (a closure over
    the register value expression), before a store fragment."""

    config: MatmulConfig
    value_transform: Any = None
    setup: tuple[str, ...] = ()
    name: str = "matmul_register_epilogue"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        if self.value_transform is None and not self.setup:
            return ""
        t = self.config.tile
        lines = list(self.setup)
        if self.value_transform is not None:
            lines += [
                "#pragma unroll",
                f"for (int i = 0; i < {t.WM}; ++i)",
                "#pragma unroll",
                f"    for (int j = 0; j < {t.WN}; ++j)",
                "#pragma unroll",
                "        for (int v = 0; v < 16; ++v)",
                f"            acc[i][j][v] = {self.value_transform('acc[i][j][v]')};",
            ]
        return "\n".join(lines)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


__all__ = [
    "MatmulAccumToDevFragment",
    "MatmulAccumToTgFragment",
    "MatmulTgToDevFragment",
    "MatmulComputeFragment",
    "MatmulConfig",
    "MatmulEpilogueStoreFragment",
    "MatmulMainloopFragment",
    "MatmulRegisterEpilogueFragment",
    "MatmulSetupFragment",
    "MatmulTileMappingFragment",
    "PersistentLoopEndFragment",
    "PersistentTiles",
    "ThreadIndexFragment",
]
