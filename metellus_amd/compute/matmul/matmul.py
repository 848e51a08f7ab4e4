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
    each workgroup paying its own launch, first load and store phases.

    ``stream_k``: when the tiles are not a multiple of P, the last partial
    round is split by k-chunks instead of by tiles (``mt_stream_k`` in the
    device library): every workgroup gets the same number of chunks, and
    tiles split between workgroups are summed through the workspace
    (``StreamKFixupFragment``).  Each loop item is a tile and a chunk range
    ``[mt_kb, mt_ke)``; in the plain loop every item is a whole tile."""

    tile_M: int
    tile_N: int
    M_dim_var: str = "M"
    N_dim_var: str = "N"
    stream_k: bool = False
    tile_K: int = 32
    K_dim_var: str = "K"
    # Row-block order instead: workgroup x takes row blocks x, x + P, ...
    # and walks all column tiles of each in order (``mt_rr_first`` /
    # ``mt_rr_last`` mark a row block's first and last tile), so a row
    # reduction in the epilogue completes inside the workgroup.
    row_blocks: bool = False


def stream_k_workspace_bytes(tile_M: int, tile_N: int, workgroups: int, anchors: int = 1) -> int:
    """Workspace of a stream-K kernel: the flag words, then one partial tile
    (every accumulator set) per workgroup."""
    return 4 * (STREAM_K_HEAD_WORDS + workgroups * tile_M * tile_N * anchors)


STREAM_K_HEAD_WORDS = 1024  # MT_WS_HEAD in the device library


@dataclass(frozen=True)
class MatmulTileMappingFragment:
    """``tg`` = (column tile, row tile) of this workgroup; with ``persistent``
    it opens the tile loop (closed by ``PersistentLoopEndFragment``) and
    defines ``mt_first_tile``, ``mt_has_next``, ``mt_next_m0/n0/kb`` and the
    item's chunk range ``mt_kb``/``mt_ke`` for the mainloop.

    ``xcd_rows`` (one tile per workgroup only): the hardware deals workgroup
    i (linear id x + gridDim.x y) to XCD i mod 8; the workgroups XCD c
    receives take row tiles c xcd_rows .. (c + 1) xcd_rows - 1, all their
    column tiles, so every A chunk is fetched into one XCD's L2 and shared
    there (gridDim.y = 8 xcd_rows)."""

    persistent: PersistentTiles | None = None
    xcd_rows: int = 0
    name: str = "tile_mapping"
    kind: str = "setup"

    @property
    def opens_tile_loop(self) -> bool:
        """LDS lifetime analysis: fragments up to the loop end run repeatedly."""
        return self.persistent is not None

    def render(self, ctx: CodegenContext) -> str:
        p = self.persistent
        if p is None and self.xcd_rows:
            return "\n".join([
                "// XCD-grouped tile order: this XCD's workgroups share their A row tiles",
                "const unsigned mt_lin = blockIdx.x + gridDim.x * blockIdx.y;",
                "const unsigned mt_slot = mt_lin / 8u;",
                f"const uint3 tg = make_uint3(mt_slot % gridDim.x, (mt_lin % 8u) * {self.xcd_rows}u + mt_slot / gridDim.x, "
                "blockIdx.z);",
            ])
        if p is None:
            return "const uint3 tg = make_uint3(blockIdx.x, blockIdx.y, blockIdx.z);"
        head = [
            f"const unsigned mt_tiles_x = ({p.N_dim_var} + {p.tile_N - 1}u) / {p.tile_N}u;",
            f"const unsigned mt_tiles = mt_tiles_x * (({p.M_dim_var} + {p.tile_M - 1}u) / {p.tile_M}u);",
            "unsigned mt_stage = 0u;  // LDS buffer holding the current k-chunk",
        ]
        if p.stream_k:
            if ctx.batched:
                raise ValueError("stream-K matmuls are not batched")
            return "\n".join(
                [
                    *head,
                    f"const unsigned mt_chunks = ({p.K_dim_var} + {p.tile_K - 1}u) / {p.tile_K}u;",
                    "mt_stream_k mt_sk;",
                    "mt_sk.init(mt_tiles, mt_chunks, gridDim.x, blockIdx.x);",
                    "for (unsigned mt_item = 0u; mt_item < mt_sk.items(); ++mt_item) {",
                    "const bool mt_first_tile = mt_item == 0u;",
                    "unsigned mt_t, mt_kb, mt_ke;",
                    "mt_sk.item(mt_item, mt_t, mt_kb, mt_ke);",
                    "const bool mt_has_next = mt_item + 1u < mt_sk.items();",
                    "unsigned mt_t_next = 0u, mt_next_kb = 0u, mt_next_ke = 0u;",
                    "if (mt_has_next) mt_sk.item(mt_item + 1u, mt_t_next, mt_next_kb, mt_next_ke);",
                    f"const unsigned mt_next_m0 = (mt_t_next / mt_tiles_x) * {p.tile_M}u;",
                    f"const unsigned mt_next_n0 = (mt_t_next % mt_tiles_x) * {p.tile_N}u;",
                    "const uint3 tg = make_uint3(mt_t % mt_tiles_x, mt_t / mt_tiles_x, blockIdx.z);",
                ]
            )
        if p.row_blocks:
            return "\n".join(
                [
                    *head,
                    f"const unsigned mt_tiles_y = ({p.M_dim_var} + {p.tile_M - 1}u) / {p.tile_M}u;",
                    "const unsigned mt_items = mt_tiles_y > blockIdx.x"
                    " ? (mt_tiles_y - blockIdx.x + gridDim.x - 1u) / gridDim.x * mt_tiles_x : 0u;",
                    "for (unsigned mt_i = 0u; mt_i < mt_items; ++mt_i) {",
                    "const unsigned mt_t = (blockIdx.x + (mt_i / mt_tiles_x) * gridDim.x) * mt_tiles_x + mt_i % mt_tiles_x;",
                    "const bool mt_first_tile = mt_i == 0u;",
                    "const bool mt_rr_first = mt_i % mt_tiles_x == 0u;",
                    "const bool mt_rr_last = mt_i % mt_tiles_x == mt_tiles_x - 1u;",
                    "const bool mt_has_next = mt_i + 1u < mt_items;",
                    "const unsigned mt_t_next = (blockIdx.x + ((mt_i + 1u) / mt_tiles_x) * gridDim.x) * mt_tiles_x"
                    " + (mt_i + 1u) % mt_tiles_x;",
                    f"const unsigned mt_next_m0 = (mt_t_next / mt_tiles_x) * {p.tile_M}u;",
                    f"const unsigned mt_next_n0 = (mt_t_next % mt_tiles_x) * {p.tile_N}u;",
                    "const unsigned mt_kb = 0u, mt_next_kb = 0u;",
                    f"const unsigned mt_ke = ({p.K_dim_var} + {p.tile_K - 1}u) / {p.tile_K}u;",
                    "const uint3 tg = make_uint3(mt_t % mt_tiles_x, mt_t / mt_tiles_x, blockIdx.z);",
                ]
            )
        return "\n".join(
            [
                *head,
                "for (unsigned mt_t = blockIdx.x; mt_t < mt_tiles; mt_t += gridDim.x) {",
                "const bool mt_first_tile = mt_t == blockIdx.x;",
                "const unsigned mt_t_next = mt_t + gridDim.x;",
                "const bool mt_has_next = mt_t_next < mt_tiles;",
                f"const unsigned mt_next_m0 = (mt_t_next / mt_tiles_x) * {p.tile_M}u;",
                f"const unsigned mt_next_n0 = (mt_t_next % mt_tiles_x) * {p.tile_N}u;",
                "const unsigned mt_kb = 0u, mt_next_kb = 0u;",
                f"const unsigned mt_ke = ({p.K_dim_var} + {p.tile_K - 1}u) / {p.tile_K}u;",
                "const uint3 tg = make_uint3(mt_t % mt_tiles_x, mt_t / mt_tiles_x, blockIdx.z);",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class StreamKFixupFragment:
    """Between a stream-K item's mainloop and its epilogue.  A contributor
    (its chunk range starts inside the tile) stores its accumulators to its
    workspace slot -- registers 4q..4q+3 of block b of lane t as one float4
    at index ``(4b + q) * NT + t``, so every store and load is one coalesced
    1 KiB row per wave -- raises its flag and
    moves on to its next item.  An owner whose range ends inside the tile
    waits for the following ranges (workgroups w-1, w-2, ...), adds their
    partials in that order, then runs the epilogue as for a whole tile."""

    config: MatmulConfig
    suffixes: tuple[str, ...] = ("",)
    name: str = "stream_k_fixup"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        t = self.config.tile
        nt = t.num_threads
        blocks = t.WM * t.WN
        tile_floats = t.tile_M * t.tile_N * len(self.suffixes)
        stores, adds = [], []
        for k, sfx in enumerate(self.suffixes):
            # quad q of block b (registers 4q..4q+3) of lane t at float4 index (b * 4 + q) * NT + t
            base = k * blocks
            loop = [
                "#pragma unroll",
                f"for (int i = 0; i < {t.WM}; ++i)",
                "#pragma unroll",
                f"    for (int j = 0; j < {t.WN}; ++j) {{",
                f"        const size_t mt_q0 = (size_t)({base}u + (unsigned)(i * {t.WN} + j)) * {4 * nt}u + threadIdx.x;",
                "#pragma unroll",
                "        for (int q = 0; q < 4; ++q) {",
            ]
            quad = f"acc{sfx}[i][j][4 * q], acc{sfx}[i][j][4 * q + 1], acc{sfx}[i][j][4 * q + 2], acc{sfx}[i][j][4 * q + 3]"
            stores += [
                *loop,
                f"            mt_part4[mt_q0 + (size_t)q * {nt}u] = mt_f32x4{{{quad}}};",
                "        }",
                "    }",
            ]
            # Per quad, a short loop over the contributors carries only that
            # quad, so the fixup's register use stays near the mainloop's and
            # nothing the mainloop keeps live is spilled for it.
            adds += [
                *loop,
                f"            mt_f32x4 mt_s = mt_f32x4{{{quad}}};",
                "            for (unsigned mt_c = 1u; mt_c <= mt_nc; ++mt_c)",
                f"                mt_s += reinterpret_cast<const mt_f32x4*>(mt_ws_part(mt_ws, blockIdx.x - mt_c, {tile_floats}u))"
                f"[mt_q0 + (size_t)q * {nt}u];",
                "#pragma unroll",
                f"            for (int e = 0; e < 4; ++e) acc{sfx}[i][j][4 * q + e] = mt_s[e];",
                "        }",
                "    }",
            ]
        return "\n".join(
            [
                "if (mt_kb != 0u) {  // contributor: hand the partial sums to the owner",
                f"    mt_f32x4* mt_part4 = reinterpret_cast<mt_f32x4*>(mt_ws_part(mt_ws, blockIdx.x, {tile_floats}u));",
                *("    " + x for x in stores),
                "    mt_sk_signal(mt_ws_flag(mt_ws, blockIdx.x));",
                "    continue;",
                "}",
                "if (mt_ke != mt_chunks) {  // owner of a split tile: add the later ranges' partial sums",
                "    const unsigned long long mt_tend = (unsigned long long)(mt_t - mt_sk.dp + 1u) * mt_chunks;",
                "    // no range is empty (stream-K needs as many units as workgroups), so the",
                "    // contributors are the workgroups at offsets 1 .. mt_nc below this one",
                "    unsigned mt_nc = 0u;",
                "    for (unsigned mt_c = mt_sk.contributor(1u, mt_tend); mt_c != 0u;"
                " mt_c = mt_sk.contributor(mt_c + 1u, mt_tend)) {",
                "        mt_sk_wait(mt_ws_flag(mt_ws, blockIdx.x - mt_c), mt_ws_error(mt_ws));",
                "        mt_nc = mt_c;",
                "    }",
                *("    " + x for x in adds),
                "}",
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
    closes_tile_loop: bool = True

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

    def render_stage(self, stage: str | None, hook: str | None = None,
                     held: tuple[str, str] | None = None) -> str:
        """MFMAs over LDS buffer ``stage`` of double-buffered tiles, or over
        single-buffered tiles when ``stage`` is None; ``hook`` names a
        callable run at each group of 4 k-steps (``mt_mfma_tile``).
        ``held`` = (group variable, has-held expression): the chunk's last
        group of 4 k-steps is carried to the next chunk
        (``mt_mfma_tile_held``; no hook)."""
        t = self.config.tile
        at, bt = self.config.a_tile_name, self.config.b_tile_name
        a_ptr = f"&{at}[{stage}][wave_m0][0]" if stage is not None else f"&{at}[wave_m0][0]"
        if t.b_layout == "nswz":  # n-major B: the wave's first column is a row
            b_ptr = f"&{bt}[{stage}][wave_n0][0]" if stage is not None else f"&{bt}[wave_n0][0]"
        else:
            b_ptr = f"&{bt}[{stage}][0][wave_n0]" if stage is not None else f"&{bt}[0][wave_n0]"
        flags = ""
        if t.a_layout != "pad" or t.b_layout == "nswz":
            aswz = "true" if t.a_layout == "swz" else "false"
            bnm = "true" if t.b_layout == "nswz" else "false"
            flags = f", {aswz}, {bnm}"
        if hook is not None and not flags:
            flags = ", false, false"
        if held is not None:
            if hook is not None:
                raise ValueError("a held group and a load hook do not combine")
            return (
                f"mt_mfma_tile_held<{t.WM}, {t.WN}, {t.tile_K}, {t.lda}, {t.ldb}{flags}>"
                f"({a_ptr}, {b_ptr}, acc{self.accumulator_suffix}, lane, {held[0]}, {held[1]});"
            )
        hook_arg = f", {hook}" if hook is not None else ""
        return (
            f"mt_mfma_tile<{t.WM}, {t.WN}, {t.tile_K}, {t.lda}, {t.ldb}{flags}>"
            f"({a_ptr}, {b_ptr}, acc{self.accumulator_suffix}, lane{hook_arg});"
        )

    def render_held_decl(self, var: str) -> str:
        """Zeroed: after a k loop that ran no chunk its flush adds 0 * 0 to
        accumulators that still hold +0."""
        t = self.config.tile
        return f"mt_mfma_group<{t.WM}, {t.WN}> {var} = {{}};"

    def render_held_flush(self, var: str) -> str:
        """The last chunk's held group, after the k loop."""
        t = self.config.tile
        return f"mt_mfma_group_run<{t.WM}, {t.WN}>({var}, acc{self.accumulator_suffix});"

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

    ``persistent`` (inside a persistent tile loop): the loop runs over the
    item's chunks ``[mt_kb, mt_ke)`` (every chunk of the tile unless a
    stream-K schedule split it); the buffer index is the running
    ``mt_stage``, flipped after every chunk of every item; only the first
    item loads its first chunk before its loop, and the last iteration of
    each item loads the next item's first chunk (``mt_next_m0/n0/kb``) into
    the other buffer, so the same one-barrier-per-chunk argument spans
    items."""

    tile_K: int
    fragments: tuple[KernelFragment, ...]
    K_dim_var: str
    persistent: bool = False
    # > 0: the next chunk's register-path loads are issued in ``spread``
    # parts at the first ``spread`` groups of 4 k-steps of the current
    # chunk's MFMAs (a hook of the first compute fragment) instead of all
    # before them; direct-to-LDS loads stay before the MFMAs unless
    # ``spread_dma``.
    spread: int = 0
    spread_dma: bool = False
    # carry each chunk's last group of 4 k-steps over the barrier into the
    # next chunk (``mt_mfma_tile_held``); not with spread loads
    held: bool = False
    name: str = "matmul_mainloop"
    kind: str = "compute"

    def _loads(self):
        return [f for f in self.fragments if hasattr(f, "render_fetch")]

    def _computes(self):
        return [f for f in self.fragments if isinstance(f, MatmulComputeFragment)]

    def _sync(self, loads) -> list[str]:
        """End of a chunk: the barrier, preceded by a wait for this wave's
        direct-to-LDS loads when there are any (the compiler does not track
        them)."""
        dma = ["__builtin_amdgcn_s_waitcnt(0);"] if any(getattr(ld, "is_dma", False) for ld in loads) else []
        return [*dma, "__syncthreads();"]

    def render(self, ctx: CodegenContext) -> str:
        loads, computes = self._loads(), self._computes()
        stages = max((ld.stages for ld in loads), default=1)
        kvar = self.K_dim_var
        tk = self.tile_K
        body: list[str] = [ld.render_decl() for ld in loads]
        if stages == 1 and any(getattr(ld, "is_dma", False) for ld in loads):
            raise ValueError("direct-to-LDS loads need double-buffered LDS tiles")
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
        sync = self._sync(loads)
        spread = self._spread(loads)
        held = self._held(spread)
        # loaders whose divisors are fixed for the tile: tested once
        plain_lds = [ld for ld in loads if getattr(ld, "plain_invariant", False)]

        def loop(plain: bool | None) -> list[str]:
            return [
                *[c.render_held_decl(f"mt_held{i}") for i, c in enumerate(computes) if held],
                "for (unsigned kt = 0; kt < n_chunks; ++kt) {",
                "    const unsigned cur = kt & 1u;",
                "    const bool more = kt + 1u < n_chunks;",
                *self._next_loads(loads, spread, persistent=False),
                *self._computes_lines(computes, spread, held, "0u"),
                *_guarded("    if (more) {",
                          [f"        {c}" for c in _nonempty(
                              ld.render_commit("cur ^ 1u", plain=plain if ld in plain_lds else None) for ld in loads)]),
                *[f"    {x}" for x in sync],
                "}",
                *self._held_flush(computes, held),
            ]

        body += [
            f"const unsigned n_chunks = ({kvar} + {tk - 1}u) / {tk}u;",
            "{",
            "    const unsigned k_chunk = 0u;",
            *[f"    {ld.render_fetch(stage='0')}" for ld in loads],
            "}",
            *_nonempty(ld.render_commit("0") for ld in loads),
            *sync,
        ]
        if plain_lds:
            # the tile's divisors are known after its first chunk: one test,
            # then a k loop whose commits carry no per-element branch (or the
            # same loop with the full chain).  all_plain is a per-wave ballot;
            # both loops hold barriers, so the choice is made workgroup-wide
            # (__syncthreads_and) and every wave enters the same loop.
            body += [
                "const bool mt_plain = __syncthreads_and(("
                + " && ".join(ld.render_plain_test() for ld in plain_lds) + ") ? 1 : 0) != 0;",
                "if (mt_plain) {",
                *[f"    {x}" for x in loop(True)],
                "} else {",
                *[f"    {x}" for x in loop(False)],
                "}",
            ]
        else:
            body += loop(None)
        return "{\n" + textwrap.indent("\n".join(body), "    ") + "\n}"

    def _held(self, spread: int) -> bool:
        if self.held and spread:
            raise ValueError("a held group and spread loads do not combine")
        return self.held and self.tile_K >= 16

    def _computes_lines(self, computes, spread: int, held: bool, k_begin: str) -> list[str]:
        """The chunk's MFMAs: with a held group (carried when kt is not the
        loop's first chunk), or with the spread loads' hook."""
        if held:
            return [f"    {c.render_stage('cur', held=(f'mt_held{i}', f'kt > {k_begin}'))}"
                    for i, c in enumerate(computes)]
        return [f"    {c.render_stage('cur', 'mt_hook' if spread and i == 0 else None)}" for i, c in enumerate(computes)]

    @staticmethod
    def _held_flush(computes, held: bool) -> list[str]:
        """After the k loop: the last chunk's held group (a zeroed group when
        the loop ran no chunk)."""
        return [c.render_held_flush(f"mt_held{i}") for i, c in enumerate(computes)] if held else []

    def _spread(self, loads) -> int:
        """Hook points the next chunk's spread loads are issued at (0: none,
        also when no loader is spread)."""
        if not self.spread or not any(self._is_spread(ld) for ld in loads):
            return 0
        return max(1, min(self.spread, self.tile_K // 8))

    def _is_spread(self, ld) -> bool:
        return self.spread_dma or not getattr(ld, "is_dma", False)

    def _next_loads(self, loads, spread: int, persistent: bool) -> list[str]:
        """Loop-head lines issuing the next chunk's loads (the next item's
        first chunk at the end of a persistent item): all of them before
        the MFMAs, or the spread ones in ``mt_hook``'s parts."""

        def guarded(lds, part, pad):
            # the next chunk of this tile (k-invariant gathers kept), or the
            # first chunk of the next item's tile (gathered afresh)
            same = [ld.render_fetch(stage="cur ^ 1u", part=part, reuse=True) for ld in lds]
            lines = ["if (more) {", f"    const unsigned k_chunk = (kt + 1u) * {self.tile_K}u;",
                     *[f"    {x}" for x in same]]
            if persistent:
                first = [ld.render_fetch(stage="cur ^ 1u", part=part) for ld in lds]
                lines += ["} else if (mt_has_next) {", "    const unsigned tile_m0 = mt_next_m0;",
                          "    const unsigned tile_n0 = mt_next_n0;",
                          f"    const unsigned k_chunk = mt_next_kb * {self.tile_K}u;", *[f"    {x}" for x in first]]
            return [pad + x for x in (*lines, "}")]

        early = [ld for ld in loads if not (spread and self._is_spread(ld))]
        out = guarded(early, None, "    ") if early else []
        if spread:
            late = [ld for ld in loads if self._is_spread(ld)]
            out += ["    const auto mt_hook = [&](int mt_q) {", f"        if (mt_q >= {spread}) return;",
                    *guarded(late, f"mt_q, {spread}", "        "), "    };"]
        return out

    def _render_persistent(self, loads, computes, body: list[str]) -> str:
        tk = self.tile_K
        sync = self._sync(loads)
        spread = self._spread(loads)
        held = self._held(spread)
        body += [
            "if (mt_first_tile) {",
            f"    const unsigned k_chunk = mt_kb * {tk}u;",
            *[f"    {ld.render_fetch(stage='mt_stage')}" for ld in loads],
            *[f"    {c}" for c in _nonempty(ld.render_commit("mt_stage") for ld in loads)],
            *[f"    {x}" for x in sync],
            "}",
            *[c.render_held_decl(f"mt_held{i}") for i, c in enumerate(computes) if held],
            "for (unsigned kt = mt_kb; kt < mt_ke; ++kt) {",
            "    const unsigned cur = mt_stage;",
            "    const bool more = kt + 1u < mt_ke;",
            *self._next_loads(loads, spread, persistent=True),
            *self._computes_lines(computes, spread, held, "mt_kb"),
            *_guarded("    if (more || mt_has_next) {",
                      [f"        {c}" for c in _nonempty(ld.render_commit("cur ^ 1u") for ld in loads)]),
            *[f"    {x}" for x in sync],
            "    mt_stage ^= 1u;",
            "}",
            *self._held_flush(computes, held),
        ]
        return "{\n" + textwrap.indent("\n".join(body), "    ") + "\n}"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    @property
    def sub_fragments(self) -> tuple[KernelFragment, ...]:
        return self.fragments


@dataclass(frozen=True)
class MatmulRowWavesFragment:
    """A whole matmul 128 columns wide on row-owning waves (``mt_rw_*``):
    256 x 128 tiles on 1024 lanes, 16 waves of 16 rows x 128 columns of
    16x16x4 MFMAs.  A wave reads its own A rows from global memory into
    registers, a 64-wide k-chunk ahead, and applies the prologue there
    (``prologue``: None; ``("transform", lambda)`` over (raw, row, col); or
    ``("gather", gather, apply, plain_apply, plain_predicate)`` with operands
    fixed per row, read once per lane); B goes straight into two LDS stages
    (``B_tile[2][64][128]``) by direct-to-LDS loads.  With a plain form of
    the prologue, every lane tests its row's divisors once
    (``__syncthreads_and``) and the workgroup runs the k loop with the plain
    form when all pass.  Needs M % 256 == 0, N == 128, K % 128 == 0 (the
    loop takes two chunks a trip).  The epilogue stores 128 bits per row;
    ``value_expr`` is a format string over ``{a0}`` with ``row`` and ``col``
    in scope."""

    a_name: str
    b_name: str
    c_name: str
    a_row_stride: int
    b_row_stride: int
    prologue: tuple | None = None
    value_expr: str | None = None
    name: str = "matmul_row_waves"
    kind: str = "compute"

    TILE_M = 256
    TILE_N = 128
    TILE_K = 64
    THREADS = 1024

    def _loop(self, pa: str) -> list[str]:
        a, b, brs = self.a_name, self.b_name, self.b_row_stride
        return [
            "for (unsigned kt = 0; kt < n_chunks; kt += 2u) {",
            "    mt_rw_load(mt_a1, mt_arow, (kt + 1u) * 64u);",
            f"    ld_B.fetch({b}, {brs}, (kt + 1u) * 64u, 0u, &B_tile[1][0][0]);",
            f"    mt_rw_chunk(mt_a0, &B_tile[0][0][0], {pa}, lane, acc);",
            "    __builtin_amdgcn_s_waitcnt(0);",
            "    __syncthreads();",
            "    if (kt + 2u < n_chunks) {",
            "        mt_rw_load(mt_a0, mt_arow, (kt + 2u) * 64u);",
            f"        ld_B.fetch({b}, {brs}, (kt + 2u) * 64u, 0u, &B_tile[0][0][0]);",
            "    }",
            f"    mt_rw_chunk(mt_a1, &B_tile[1][0][0], {pa}, lane, acc);",
            "    __builtin_amdgcn_s_waitcnt(0);",
            "    __syncthreads();",
            "}",
        ]

    def render(self, ctx: CodegenContext) -> str:
        a, b, c = self.a_name, self.b_name, self.c_name
        pro = self.prologue
        lines = [
            "const unsigned lane = mt_lane();",
            "const unsigned wave = mt_wave();",
            "const unsigned tile_m0 = blockIdx.y * 256u;",
            "const unsigned mt_row = tile_m0 + wave * 16u + (lane & 15u);",
            "mt_f32x4 acc[8];",
            "#pragma unroll",
            "for (int j = 0; j < 8; ++j) acc[j] = mt_f32x4{0.f, 0.f, 0.f, 0.f};",
            f"const mt_tile_dma<64, 128, 1024, false> ld_B({self.b_row_stride}, threadIdx.x);",
            f"const float* __restrict__ mt_arow = {a} + (size_t)mt_row * {self.a_row_stride}u + 16u * (lane >> 4);",
            "mt_f32x4 mt_a0[4], mt_a1[4];",
        ]
        plain = False
        if pro is None:
            lines.append("const auto mt_pa = [](float raw) -> float { return raw; };")
        elif pro[0] == "transform":
            lines += [f"const auto xt = {pro[1]};",
                      "const auto mt_pa = [=](float raw) -> float { return xt(raw, mt_row, 0u); };"]
        else:
            _, gather, apply, plain_apply, plain_pred = pro
            lines += [f"const auto xg = {gather};", f"const auto xa = {apply};",
                      "const auto mt_e = xg(mt_row, 0u);  // the row's operands",
                      "const auto mt_pa = [=](float raw) -> float { return xa(raw, mt_e); };"]
            if plain_apply is not None:
                plain = True
                lines += [f"const auto xq = {plain_apply};", f"const auto xp = {plain_pred};",
                          "const auto mt_pq = [=](float raw) -> float { return xq(raw, mt_e); };"]
        lines += [
            "mt_rw_load(mt_a0, mt_arow, 0u);",
            f"ld_B.fetch({b}, {self.b_row_stride}, 0u, 0u, &B_tile[0][0][0]);",
            "__builtin_amdgcn_s_waitcnt(0);",
            "__syncthreads();",
            "const unsigned n_chunks = K / 64u;",
        ]
        if plain:
            lines += ["if (__syncthreads_and(xp(mt_e) ? 1 : 0) != 0) {",
                      *[f"    {x}" for x in self._loop("mt_pq")], "} else {",
                      *[f"    {x}" for x in self._loop("mt_pa")], "}"]
        else:
            lines += self._loop("mt_pa")
        value = self.value_expr.format(a0="acc[4 * h + j][i]") if self.value_expr else "acc[4 * h + j][i]"
        lines += [
            "#pragma unroll",
            "for (int i = 0; i < 4; ++i) {",
            "    const unsigned row = tile_m0 + wave * 16u + 4u * (lane >> 4) + (unsigned)i;",
            "#pragma unroll",
            "    for (int h = 0; h < 2; ++h) {",
            "        const unsigned col0 = 64u * (unsigned)h + 4u * (lane & 15u);",
            "        mt_f32x4 mt_o;",
            "#pragma unroll",
            "        for (int j = 0; j < 4; ++j) {",
            "            const unsigned col = col0 + (unsigned)j;",
            "            (void)col;",
            f"            mt_o[j] = {value};",
            "        }",
            f"        *reinterpret_cast<mt_f32x4*>(&{c}[(size_t)row * N + col0]) = mt_o;",
            "    }",
            "}",
        ]
        return "{\n" + textwrap.indent("\n".join(lines), "    ") + "\n}"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return (TgmemAccess("B_tile", "read", 2 * 64 * 128, (2, 64, 128)),)


# K-resident row waves: the previous chunk's right half is stored one row
# after every KR_STORE_STRIDE-th MFMA group of this chunk's left half (1:
# after each of the first four groups); this chunk's left half one row after
# each of the first four groups of its right half.  KR_STORE_POLICY is the
# buffer stores' cache-policy operand (0: default; 16: sc1, device scope,
# written through the L2).  Measured on C5 S (32 heads, medians of 25-30
# launches, one box):
# stores after the chunk's MFMAs 263.4 us; one row per group of the other
# half 255.1; spread over every other group of the left half 251.2; sc1
# 246.7; the right half's stores in the first four groups 245.6 (0.889 of
# the fp32 MFMA peak).  Without any stores: 239.7.  Per chunk 14.8 us
# against 13.6 of MFMA work, plus ~13 us fixed (launch, first loads, last
# stores).  The first chunk waits for all of A as well as its B: a partial
# vmcnt counting only the A loads issued after the B chunk is not a safe
# wait for that chunk (direct-to-LDS loads and ordinary loads do not
# retire in issue order), and it gained under 1 us.
KR_STORE_STRIDE = 2
KR_STORE_POLICY = 16


@dataclass(frozen=True)
class MatmulKResidentFragment:
    """A matmul with a short K (64 or 128) and an n-major B (read along K,
    such as the transposed view K^T) on K-resident row waves (``mt_kr_*``):
    1024 lanes own 256 rows, each wave 16 of them, whose whole K sits in its
    registers (loaded once; the prologue applied there).  The workgroup walks
    ``chunks`` 128-column chunks of B, staged by direct-to-LDS loads in two
    LDS stages ``B_tile[2][128][K]``; every chunk is a finished 256 x 128
    output tile on 16x16x4 MFMAs, walked column half by column half.  Its
    stores (128 bits per row) go out between MFMAs: one row of the
    previous chunk's right half after each of the first 4 MFMA groups of
    this chunk's left half, one row of this chunk's left half after each of
    the first 4 groups of its right half (the halves use disjoint
    accumulators, so no register holds a result longer).  Workgroup (x, y) takes rows
    256 y .. 256 y + 255 and columns 128 chunks x onwards.  ``prologue``:
    None, ``("transform", lambda)`` over (raw, row, col), or
    ``("gather", gather, apply)`` with operands fixed per row.
    ``value_expr``: a format string over ``{a0}`` with ``row`` and ``col`` in
    scope.  Needs M % 256 == 0, N % (128 chunks) == 0 and an output (one
    program's) below 2 GiB: stores address it by 32-bit byte offsets.

    ``reduction`` = (op, red_name): the kernel also reduces every output row
    (after the epilogue) into ``red_name[row]``; the workgroup then walks
    whole rows (one column group).  Each lane folds its values of each of
    its 4 rows in column order (chunk, then column half, then column), and
    the 16 lanes sharing a row combine by xor-butterfly over lane bits 0..3,
    low bit first -- one fixed order, the same for every batch size."""

    a_name: str
    b_name: str
    c_name: str
    a_row_stride: int
    b_col_stride: int
    K: int
    chunks: int
    prologue: tuple | None = None
    value_expr: str | None = None
    reduction: tuple[str, str] | None = None
    name: str = "matmul_k_resident"
    kind: str = "compute"

    TILE_M = 256
    TILE_N = 128
    THREADS = 1024

    def _prologue_lines(self) -> list[str]:
        pro, K = self.prologue, self.K
        if pro is None:
            return []
        if pro[0] == "transform":
            lines = [f"const auto xt = {pro[1]};"]
            apply = "xt(mt_a[q][e], mt_row, mt_k0 + 4u * (unsigned)q + (unsigned)e)"
        else:
            _, gather, app = pro[:3]
            lines = [f"const auto xg = {gather};", f"const auto xa = {app};",
                     "const auto mt_e = xg(mt_row, 0u);  // the row's operands"]
            apply = "xa(mt_a[q][e], mt_e)"
        return lines + [
            f"const unsigned mt_k0 = {K // 4}u * (lane >> 4);",
            "(void)mt_k0;",
            "#pragma unroll",
            f"for (int q = 0; q < {K // 16}; ++q)",
            "#pragma unroll",
            f"    for (int e = 0; e < 4; ++e) mt_a[q][e] = {apply};",
        ]

    def render(self, ctx: CodegenContext) -> str:
        a, b, c, K = self.a_name, self.b_name, self.c_name, self.K
        if K not in (64, 128):
            raise ValueError(f"K-resident rows hold K = 64 or 128; got {K}")
        bcs = self.b_col_stride
        value = self.value_expr.format(a0="acc[4 * h + j][i]") if self.value_expr else "acc[4 * h + j][i]"
        red = self.reduction
        opc, ident = _RR_OPS[red[0]] if red is not None else (None, None)
        T = K // 16
        # the previous right half: one row every st groups of the left half
        st = max(1, min(KR_STORE_STRIDE, T // 4))
        lines = [
            "const unsigned lane = mt_lane();",
            "const unsigned wave = mt_wave();",
            "const unsigned tile_m0 = blockIdx.y * 256u;",
            f"const unsigned mt_n0 = blockIdx.x * {128 * self.chunks}u;",
            "const unsigned mt_row = tile_m0 + wave * 16u + (lane & 15u);",
            f"const mt_kr_dma<{K}, 1024> ld_B({bcs}u, threadIdx.x);",
            f"ld_B.fetch({b}, {bcs}u, mt_n0, &B_tile[0][0][0]);",
            f"const float* __restrict__ mt_arow = {a} + (size_t)mt_row * {self.a_row_stride}u + {K // 4}u * (lane >> 4);",
            f"mt_f32x4 mt_a[{T}];",
            "#pragma unroll",
            f"for (int q = 0; q < {T}; ++q) mt_a[q] = mt_ld4(mt_arow + 4u * (unsigned)q);",
            *self._prologue_lines(),
            "mt_f32x4 acc[8];",
            "#pragma unroll",
            "for (int j = 0; j < 8; ++j) acc[j] = mt_f32x4{0.f, 0.f, 0.f, 0.f};",
            *([f"float mt_red[4] = {{{ident}, {ident}, {ident}, {ident}}};"] if red is not None else []),
            "// row i of a finished column half h (blocks 4h .. 4h + 3) of the chunk",
            "// at columns col_base: the epilogue, then one 128-bit buffer store at",
            "// this lane's byte offset plus a wave-uniform one",
            f"const mt_u32x4 mt_rs = mt_raw_buffer({c}, M * N * 4u);",
            "const unsigned mt_voff = ((tile_m0 + wave * 16u + 4u * (lane >> 4)) * N + mt_n0 + 4u * (lane & 15u)) * 4u;",
            "const auto mt_store_row = [&](int h, int i, unsigned col_base) {",
            "    const unsigned row = tile_m0 + wave * 16u + 4u * (lane >> 4) + (unsigned)i;",
            "    const unsigned col0 = col_base + 64u * (unsigned)h + 4u * (lane & 15u);",
            "    mt_f32x4 mt_o;",
            "#pragma unroll",
            "    for (int j = 0; j < 4; ++j) {",
            "        const unsigned col = col0 + (unsigned)j;",
            "        (void)col;",
            f"        mt_o[j] = {value};",
            *([f"        mt_red[i] = mt_rr_op<{opc}>(mt_red[i], mt_o[j]);"] if red is not None else []),
            "    }",
            f"    mt_buffer_store4<{KR_STORE_POLICY}>(mt_o, mt_rs, mt_voff, "
            "((unsigned)i * N + (col_base - mt_n0) + 64u * (unsigned)h) * 4u);",
            "};",
            "__builtin_amdgcn_s_waitcnt(0);",
            "__syncthreads();",
            f"for (unsigned ch = 0; ch < {self.chunks}u; ++ch) {{",
            f"    if (ch + 1u < {self.chunks}u) ld_B.fetch({b}, {bcs}u, mt_n0 + (ch + 1u) * 128u, "
            "&B_tile[(ch + 1u) & 1u][0][0]);",
            "    const unsigned col_base = mt_n0 + ch * 128u;",
            "    // while the left half's MFMAs run: the previous chunk's right half,",
            "    // one row per group; while the right half's run: this chunk's left",
            "    const auto mt_hook = [&](int q) {",
            f"        if (q < {4 * st} && q % {st} == 0) {{",
            f"            if (ch > 0u) mt_store_row(1, q / {st}, col_base - 128u);",
            f"            if (q == {3 * st}) {{",
            "#pragma unroll",
            "                for (int j = 4; j < 8; ++j) acc[j] = mt_f32x4{0.f, 0.f, 0.f, 0.f};",
            "            }",
            f"        }} else if (q >= {T} && q < {T + 4}) {{",
            f"            mt_store_row(0, q - {T}, col_base);",
            f"            if (q == {T + 3}) {{",
            "#pragma unroll",
            "                for (int j = 0; j < 4; ++j) acc[j] = mt_f32x4{0.f, 0.f, 0.f, 0.f};",
            "            }",
            "        }",
            "    };",
            f"    mt_kr_chunk<{K}>(mt_a, &B_tile[ch & 1u][0][0], lane, acc, mt_hook);",
            "    // the next chunk's B has landed (and the stores issued a half",
            "    // chunk ago have drained)",
            "    __builtin_amdgcn_s_waitcnt(0);",
            "    __syncthreads();",
            "}",
            "// the last chunk's right half",
            "#pragma unroll",
            f"for (int i = 0; i < 4; ++i) mt_store_row(1, i, mt_n0 + {128 * (self.chunks - 1)}u);",
        ]
        if red is not None:
            lines += [
                "// the 16 lanes holding a row: xor-butterfly over lane bits 0..3",
                "#pragma unroll",
                "for (int i = 0; i < 4; ++i) {",
                f"    mt_red[i] = mt_rr_op<{opc}>(mt_red[i], mt_xor_lanes<1u>(mt_red[i]));",
                f"    mt_red[i] = mt_rr_op<{opc}>(mt_red[i], mt_xor_lanes<2u>(mt_red[i]));",
                f"    mt_red[i] = mt_rr_op<{opc}>(mt_red[i], mt_xor_lanes<4u>(mt_red[i]));",
                f"    mt_red[i] = mt_rr_op<{opc}>(mt_red[i], mt_xor_lanes<8u>(mt_red[i]));",
                "}",
                "if ((lane & 15u) == 0u) {",
                "    const unsigned row0 = tile_m0 + wave * 16u + 4u * (lane >> 4);",
                "#pragma unroll",
                f"    for (int i = 0; i < 4; ++i) {red[1]}[row0 + (unsigned)i] = mt_red[i];",
                "}",
            ]
        return "{\n" + textwrap.indent("\n".join(lines), "    ") + "\n}"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return (TgmemAccess("B_tile", "read", 2 * 128 * self.K, (2, 128, self.K)),)


def _nonempty(lines) -> list[str]:
    return [x for x in lines if x]


def _guarded(head: str, lines: list[str]) -> list[str]:
    """``head`` ... ``}`` around ``lines``, or nothing when there are none."""
    return [head, *lines, "    }"] if lines else []


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


_RR_OPS = {"sum": (0, "0.0f"), "max": (1, "(-INFINITY)"), "min": (2, "INFINITY"), "product": (3, "1.0f")}


@dataclass(frozen=True)
class MatmulRowReduceStoreFragment:
    """(Extension: the matmul -> reduction epilogue.)  Store the tile like
    ``MatmulEpilogueStoreFragment``, then reduce each of its rows with
    ``op`` into ``red_name[row]`` across the tiles of the row:

    * the workgroup's previous tile, if any, is published first
      (``mt_rr_finish``): its writes completed during this tile's mainloop,
      so the publish does not wait for this tile's stores;
    * the stored values (columns beyond N: the op's identity) are combined
      per wave by ``mt_wave_row_reduce``, then over the ``sg_N`` waves that
      share rows through LDS ``row_red`` in wave order;
    * the tile's row values go to the workspace after its flag words, at
      row block ``blockIdx.z * tiles_m + tile_m0 / tile_M`` and column tile
      ``tile_n0 / tile_N``; the tile becomes the pending one, published by the
      next tile or by ``MatmulRowReduceFinishFragment`` after the last.

    Flag word ``block`` counts the published tiles of the block; the
    workgroup that completes it combines its tiles in column order.  The
    workspace holds ``rr_workspace_bytes`` and at most MT_WS_HEAD - 1 row
    blocks (the assembler checks).  ``MatmulRowReduceSetupFragment`` declares
    the pending tile before the tile loop."""

    config: MatmulConfig
    op: str
    red_name: str
    value_expr: str | None = None
    check: bool = False
    lds_name: str = "row_red"
    # the tile loop walks whole row blocks (PersistentTiles.row_blocks):
    # lane t < tile_M carries row t's running value from tile to tile and
    # writes it after the block's last tile -- no workspace, no publish
    local: bool = False
    name: str = "matmul_row_reduce_store"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        t, cfg = self.config.tile, self.config
        opi, ident = _RR_OPS[self.op]
        M, N = cfg.M_dim_var, cfg.N_dim_var
        value = self.value_expr.format(a0="acc[i][j][v]") if self.value_expr else "acc[i][j][v]"
        guard = f"if (row < {M} && col < {N}) " if self.check else ""
        keep_col = f"col < {N} ? mt_y : {ident}" if self.check else "mt_y"
        keep = max(1, 16 * t.WM // 32)
        tm, tn, sgn, rr = t.tile_M, t.tile_N, t.sg_N, self.lds_name
        combine = _rr_combine(self.op)
        if self.local:
            if tm > t.num_threads:
                raise ValueError("a local row reduction keeps one row per lane: tile_M <= lanes")
            tail = [
                f"    if (threadIdx.x < {tm}u) {{",
                f"        float r = {rr}[0][threadIdx.x];",
                *(f"        r = {combine('r', f'{rr}[{n}][threadIdx.x]')};" for n in range(1, sgn)),
                f"        mt_rr_run = mt_rr_first ? r : {combine('mt_rr_run', 'r')};",
                f"        if (mt_rr_last && tile_m0 + threadIdx.x < {M}) {self.red_name}[tile_m0 + threadIdx.x] = mt_rr_run;",
                "    }",
            ]
        else:
            tail = [
                f"    mt_rr_pend = blockIdx.z * (({M} + {tm - 1}u) / {tm}u) + tile_m0 / {tm}u;",
                "    mt_rr_pend_m0 = tile_m0;",
                f"    float* mt_rr_part = mt_ws + MT_WS_HEAD + (size_t)mt_rr_pend * (({N} + {tn - 1}u) / {tn}u) * {tm}u;",
                f"    for (unsigned t = threadIdx.x; t < {tm}u; t += {t.num_threads}u) {{",
                f"        float r = {rr}[0][t];",
                *(f"        r = {combine('r', f'{rr}[{n}][t]')};" for n in range(1, sgn)),
                f"        mt_rr_part[(size_t)(tile_n0 / {tn}u) * {tm}u + t] = r;",
                "    }",
            ]
        return "\n".join(
            [
                "" if self.local else _rr_finish_call(self, "if (mt_rr_pend != 0xffffffffu) "),
                "#pragma unroll",
                f"for (int i = 0; i < {t.WM}; ++i) {{",
                "#pragma unroll",
                f"    for (int j = 0; j < {t.WN}; ++j) {{",
                "        const unsigned col = tile_n0 + wave_n0 + (unsigned)j * 32u + (lane & 31u);",
                "#pragma unroll",
                "        for (int v = 0; v < 16; ++v) {",
                "            const unsigned row = tile_m0 + wave_m0 + (unsigned)i * 32u + mt_acc_row(v, lane);",
                f"            const float mt_y = {value};",
                f"            {guard}{cfg.c_buffer_name}[(size_t)row * {N} + col] = mt_y;",
                f"            acc[i][j][v] = {keep_col};",
                "        }",
                "    }",
                "}",
                "{",
                f"    float mt_rr_keep[{keep}];",
                f"    mt_wave_row_reduce<{t.WM}, {t.WN}, {opi}>(acc, lane, mt_rr_keep);",
                "#pragma unroll",
                f"    for (int k = 0; k < {keep}; ++k)",
                f"        {rr}[wave % {sgn}u][wave_m0 + mt_rr_row<{t.WM}>(lane, k)] = mt_rr_keep[k];",
                "    __syncthreads();",
                *tail,
                "}",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        shape = rr_lds_shape(self.config.tile)
        return (
            TgmemAccess(self.lds_name, "write", _prod(shape), shape),
            TgmemAccess(self.lds_name, "read", _prod(shape), shape),
        )


def _rr_finish_call(frag: "MatmulRowReduceStoreFragment", head: str) -> str:
    t, cfg = frag.config.tile, frag.config
    opi, _ = _RR_OPS[frag.op]
    return (
        f"{head}mt_rr_finish<{opi}, {t.tile_M}u, {t.num_threads}u>(mt_ws, mt_rr_pend, "
        f"({cfg.N_dim_var} + {t.tile_N - 1}u) / {t.tile_N}u, mt_rr_pend_m0, {cfg.M_dim_var}, {frag.red_name}, "
        f"reinterpret_cast<unsigned*>(&{frag.lds_name}[{t.sg_N}][0]));"
    )


@dataclass(frozen=True)
class MatmulRowReduceSetupFragment:
    """Declares the pending tile of the row-reduction epilogue (none yet),
    or in the local form the running row value; placed before the tile
    loop."""

    local: bool = False
    name: str = "matmul_row_reduce_setup"
    kind: str = "compute"

    def render(self, ctx: CodegenContext) -> str:
        if self.local:
            return "float mt_rr_run = 0.0f;  // this lane's row: the row block's value so far"
        return "unsigned mt_rr_pend = 0xffffffffu, mt_rr_pend_m0 = 0u;  // row block of the unpublished tile"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


@dataclass(frozen=True)
class MatmulRowReduceFinishFragment:
    """Publishes the workgroup's last tile of the row-reduction epilogue;
    placed after the tile loop (every workgroup has at least one tile)."""

    store: MatmulRowReduceStoreFragment
    name: str = "matmul_row_reduce_finish"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        return _rr_finish_call(self.store, "if (mt_rr_pend != 0xffffffffu) ")

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        shape = rr_lds_shape(self.store.config.tile)
        return (
            TgmemAccess(self.store.lds_name, "write", _prod(shape), shape),
            TgmemAccess(self.store.lds_name, "read", _prod(shape), shape),
        )


def _rr_combine(op: str):
    fn = {"sum": "{a} + {b}", "max": "fmaxf({a}, {b})", "min": "fminf({a}, {b})", "product": "{a} * {b}"}[op]
    return lambda a, b: fn.format(a=a, b=b)


def rr_lds_shape(t: TileConfig) -> tuple[int, int]:
    """LDS of the row-reduction epilogue: one row of tile_M values per wave
    column, and one more row whose first word is the publish flag."""
    return (t.sg_N + 1, t.tile_M)


def rr_workspace_bytes(M: int, N: int, t: TileConfig, batch: int = 1) -> int:
    """Workspace of the row-reduction epilogue: the flag words, then one
    tile_M-value row per (program, row block, column tile)."""
    blocks = batch * ((M + t.tile_M - 1) // t.tile_M)
    return 4 * (STREAM_K_HEAD_WORDS + blocks * ((N + t.tile_N - 1) // t.tile_N) * t.tile_M)


def rr_row_blocks(M: int, t: TileConfig, batch: int = 1) -> int:
    return batch * ((M + t.tile_M - 1) // t.tile_M)


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
    "MatmulRowWavesFragment",
    "MatmulAccumToTgFragment",
    "MatmulTgToDevFragment",
    "MatmulComputeFragment",
    "MatmulConfig",
    "MatmulEpilogueStoreFragment",
    "MatmulMainloopFragment",
    "MatmulRegisterEpilogueFragment",
    "MatmulRowReduceFinishFragment",
    "MatmulRowReduceSetupFragment",
    "MatmulRowReduceStoreFragment",
    "MatmulSetupFragment",
    "MatmulTileMappingFragment",
    "PersistentLoopEndFragment",
    "PersistentTiles",
    "ThreadIndexFragment",
]
