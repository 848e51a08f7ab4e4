"""Cooperative global <-> LDS tile movement for gfx950.

``TgLoadFragment`` keeps the reference's parameters (reference:
src/memory/memory.py:434-475): a ``tile_shape`` tile of the strided source
``src[(row_start + r)*row_stride + (col_start + c)*col_stride]`` lands in LDS
tile ``dst_name``; elements outside ``(row_limit, col_limit)`` read as 0.0
and ``value_transform`` (an elementwise prologue) applies to in-bounds
elements only (reference: memory.py:8-11).

gfx950 choices (in ``mt_device.h``):

* loads are 128-bit along whichever axis is contiguous in the source --
  columns (``mt_tile_colvec``) or rows (``mt_tile_rowvec``, e.g. a K^T view)
  -- else one element per load (``mt_tile_scalar``);
* a load is split into ``fetch`` (global -> registers) and ``commit``
  (registers -> LDS) so a pipelined mainloop can keep the next tile's loads
  in flight during the MFMAs; LDS tiles may hold ``stages`` buffers and a
  padded row pitch;
* when the mode is not given, it is chosen from what the parameters prove:
  128-bit loads without run-time checks need an integer row stride and
  column limit that are multiples of 4; a contiguous row with a symbolic
  stride or limit gets ``colvec_safe`` (128-bit where a run-time check shows
  the 4 columns aligned and in bounds, else per element), as the reference
  does (memory.py:277-286);
* without ``dst_pitch`` the LDS row pitch is the declared array's
  (``sizeof(dst[0]) / sizeof(float)``), so a padded declaration works;
* lane index: ``threadIdx.x`` for one-dimensional workgroups, the flat
  ``threadIdx.y * tg_x + threadIdx.x`` when the context has ``tg_y > 1``.

The transform, when present, is rendered as a C++ lambda
``(float raw, unsigned global_row, unsigned global_col) -> float``; a
reference-style ``value_transform`` closure (raw expression -> expression
over ``global_row``/``global_col``) is wrapped into one.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess

ValueTransform = Callable[[str], str]


def flat_tid(ctx: CodegenContext) -> str:
    """This lane's index within the workgroup."""
    return f"(threadIdx.y * {ctx.tg_x}u + threadIdx.x)" if ctx.tg_y > 1 else "threadIdx.x"


def _mult4(limit: str | None) -> bool:
    """A bound that is absent or a literal multiple of 4."""
    return limit is None or (_is_int(limit) and int(limit) % 4 == 0)


def _is_int(s: str) -> bool:
    try:
        int(s)
    except (TypeError, ValueError):
        return False
    return True


def dma_offsets_fit(rows: int, cols: int, row_stride) -> bool:
    """A direct-to-LDS loader keeps each lane's byte offset from the tile
    origin in 32 bits (``mt_tile_dma``): the row stride must be a literal and
    the farthest element of a rows x cols tile within 2^32 bytes."""
    if not _is_int(str(row_stride)):
        return False
    return ((rows - 1) * int(row_stride) + cols) * 4 < 1 << 32


@dataclass(frozen=True)
class TgLoadFragment:
    name: str
    src_name: str
    src_row_stride: str
    row_start: str
    col_start: str
    dst_name: str
    tile_shape: tuple[int, int]
    num_threads: int
    row_limit: str | None = None
    col_limit: str | None = None
    src_col_stride: str = "1"
    value_transform: ValueTransform | None = None
    kind: str = "memory"
    # gfx950 layout controls
    dst_pitch: int | None = None
    stages: int = 1
    mode: str | None = None  # "colvec" | "rowvec" | "scalar" | "dma" (default: from strides)
    transform_lambda: str | None = None
    # Apply the transform when the registers are written to LDS rather than
    # when the loads return, so a pipelined mainloop does not wait for the
    # next chunk's loads before its MFMAs.  Worth it when the transform reads
    # only small broadcast operands (those loads then happen at commit).
    defer_transform: bool = False
    # Gather / apply: the transform's external operands are loaded with the
    # tile (``gather_lambda``: (row, col) -> mt_vals<n_gathered>) and the
    # chain (``apply_lambda``: (raw, operands) -> float) runs at commit.
    gather_lambda: str | None = None
    apply_lambda: str | None = None
    n_gathered: int = 0
    # The gathered operands are constant along the loader's vector axis (a
    # column broadcast for "colvec", a row broadcast for "rowvec"): gather
    # them once per 128-bit slot.
    gather_per_slot: bool = False
    # The per-slot operands are also constant along the matmul's k axis (the
    # loader walks k along its vector axis), so every k-chunk of one output
    # tile needs the same ones: they are gathered with a tile's first chunk
    # and kept for the rest (``render_fetch(reuse=True)``: fetch_keep).
    gather_invariant: bool = False
    # With gathering: the chain with its divisions reduced to x * 1/y
    # (``plain_apply_lambda``) and the test that makes it exact
    # (``plain_predicate``, over the gathered operands); the commit takes the
    # plain chain when the whole wave passes (commit_apply_fast).
    plain_apply_lambda: str | None = None
    plain_predicate: str | None = None
    # mode "dma": direct-to-LDS loads (mt_tile_dma) of a row-major source
    # (row stride src_row_stride, unit column stride, every element in
    # bounds, no transform) into a dense tile of tile_shape; the fetch
    # writes LDS stage ``stage`` itself and there is no commit.  The
    # consumer waits for the loads (s_waitcnt) before its barrier.
    # ``dma_swizzle`` permutes each row's 16-byte slots (mt_swz).
    dma_swizzle: bool = False

    @property
    def pitch(self) -> str:
        """LDS row pitch in floats (a C++ constant expression)."""
        if self.dst_pitch is not None:
            return str(self.dst_pitch)
        row = f"{self.dst_name}[0][0]" if self.stages > 1 else f"{self.dst_name}[0]"
        return f"sizeof({row}) / sizeof(float)"

    @property
    def check(self) -> bool:
        return self.row_limit is not None or self.col_limit is not None

    def resolved_mode(self) -> str:
        if self.mode is not None:
            return self.mode
        rows, cols = self.tile_shape
        rs, cs = self.src_row_stride, self.src_col_stride
        pitch_ok = self.dst_pitch is None or self.dst_pitch % 4 == 0
        if cs == "1" and cols % 4 == 0 and pitch_ok:
            proven = _is_int(rs) and int(rs) % 4 == 0 and _mult4(self.col_limit)
            return "colvec" if proven else "colvec_safe"
        if rs == "1" and rows % 4 == 0 and _is_int(cs) and int(cs) % 4 == 0 and _mult4(self.row_limit):
            return "rowvec"
        return "scalar"

    @property
    def loader(self) -> str:
        return f"ld_{self.dst_name}"

    @property
    def xform(self) -> str:
        return f"xf_{self.dst_name}"

    def _lambda(self) -> str:
        if self.transform_lambda is not None:
            return self.transform_lambda
        if self.value_transform is not None:
            expr = self.value_transform("raw")
            return f"[=](float raw, unsigned global_row, unsigned global_col) -> float {{ return {expr}; }}"
        return "mt_identity{}"

    @property
    def gathering(self) -> bool:
        return self.gather_lambda is not None

    @property
    def is_dma(self) -> bool:
        return self.mode == "dma"

    def _check_dma(self) -> None:
        rows, cols = self.tile_shape
        if self.check or self._has_transform() or self.gathering or self.src_col_stride != "1":
            raise ValueError(f"{self.name}: direct-to-LDS loads need an unmasked, untransformed row-major source")
        if self.stages < 2 or (self.dst_pitch is not None and self.dst_pitch != cols):
            raise ValueError(f"{self.name}: direct-to-LDS loads fill a dense, double-buffered tile")
        slots = rows * cols // 4
        if cols % 4 or slots % 64 or (slots // 64) % (self.num_threads // 64):
            raise ValueError(f"{self.name}: a {rows}x{cols} tile does not split into whole wave loads")
        if not dma_offsets_fit(rows, cols, self.src_row_stride):
            raise ValueError(f"{self.name}: a {rows}x{cols} tile at row stride {self.src_row_stride} needs "
                             "per-lane offsets beyond 32 bits")

    def render_decl(self) -> str:
        rows, cols = self.tile_shape
        mode = self.resolved_mode()
        if mode == "dma":
            self._check_dma()
            swz = "true" if self.dma_swizzle else "false"
            return (f"const mt_tile_dma<{rows}, {cols}, {self.num_threads}, {swz}> "
                    f"{self.loader}({self.src_row_stride}, threadIdx.x);")
        tmpl = {"colvec": "mt_tile_colvec", "colvec_safe": "mt_tile_colvec", "rowvec": "mt_tile_rowvec",
                "scalar": "mt_tile_scalar"}[mode]
        if self.gathering:
            if mode == "colvec_safe" or self.apply_lambda is None or self.n_gathered < 1:
                raise ValueError(f"{self.name}: gather/apply needs a proven load mode and an apply lambda")
            if self.gather_per_slot and mode not in ("colvec", "rowvec"):
                raise ValueError(f"{self.name}: per-slot gathers need a vectorised load mode")
            if self.gather_invariant and not self.gather_per_slot:
                raise ValueError(f"{self.name}: k-invariant gathers are per-slot gathers")
            slot = ", true" if self.gather_per_slot else ""
            plain = ""
            if self._plain_commit(mode):
                plain = (f"\nconst auto xq_{self.dst_name} = {self.plain_apply_lambda};"
                         f"\nconst auto xp_{self.dst_name} = {self.plain_predicate};")
            return (
                f"{tmpl}_g<{rows}, {cols}, {self.num_threads}, {self.n_gathered}{slot}> {self.loader};\n"
                f"const auto xg_{self.dst_name} = {self.gather_lambda};\n"
                f"const auto xa_{self.dst_name} = {self.apply_lambda};{plain}"
            )
        return f"{tmpl}<{rows}, {cols}, {self.num_threads}> {self.loader};\nconst auto {self.xform} = {self._lambda()};"

    def render_fetch(
        self, tid: str = "threadIdx.x", stage: str | None = None, part: str | None = None, reuse: bool = False
    ) -> str:
        """The loads of one tile; ``stage`` is the LDS buffer a direct-to-LDS
        loader writes (register loaders write at commit and ignore it).
        ``part`` = "q, Q": only the loads of part q of Q (``mt_in_part``).
        ``reuse``: a later chunk of the same output tile -- a loader with
        k-invariant gathered operands keeps them (``fetch_keep``)."""
        if reuse and self.gathering and self.gather_invariant:
            check = "true" if self.check else "false"
            rlim = self.row_limit if self.row_limit is not None else "0xffffffffu"
            clim = self.col_limit if self.col_limit is not None else "0xffffffffu"
            strides = self.src_row_stride if self.resolved_mode() == "colvec" else self.src_col_stride
            text = (
                f"{self.loader}.template fetch_keep<{check}>({self.src_name}, {strides}, {self.row_start}, "
                f"{self.col_start}, {rlim}, {clim}, {tid});"
            )
        else:
            text = self._render_fetch(tid, stage)
        if part is not None:
            assert text.endswith(");")
            text = f"{text[:-2]}, {part});"
        return text

    def _render_fetch(self, tid: str, stage: str | None) -> str:
        if self.is_dma:
            if stage is None:
                raise ValueError(f"{self.name}: a direct-to-LDS fetch needs its LDS stage")
            return (
                f"{self.loader}.fetch({self.src_name}, {self.src_row_stride}, {self.row_start}, "
                f"{self.col_start}, {self.stage_ptr(stage)});"
            )
        rlim = self.row_limit if self.row_limit is not None else "0xffffffffu"
        clim = self.col_limit if self.col_limit is not None else "0xffffffffu"
        check = "true" if self.check else "false"
        mode = self.resolved_mode()
        deferred = self.defer_transform and self._has_transform() and mode != "colvec_safe"
        if self.gathering:
            head = f"{self.loader}.template fetch_gather<{check}>({self.src_name}, "
            deferred = False
        elif mode == "colvec_safe":
            head = f"{self.loader}.fetch_safe({self.src_name}, "
        else:
            verb = "fetch_raw" if deferred else "fetch"
            head = f"{self.loader}.template {verb}<{check}>({self.src_name}, "
        if mode in ("colvec", "colvec_safe"):
            strides = f"{self.src_row_stride}"
        elif mode == "rowvec":
            strides = f"{self.src_col_stride}"
        else:
            strides = f"{self.src_row_stride}, {self.src_col_stride}"
        if self.gathering:
            tail = f", xg_{self.dst_name})"
        else:
            tail = ")" if deferred else f", {self.xform})"
        return f"{head}{strides}, {self.row_start}, {self.col_start}, {rlim}, {clim}, {tid}{tail};"

    @property
    def plain_invariant(self) -> bool:
        """A plain chain whose divisors stay the same for every k-chunk of a
        tile (k-invariant gathers): one test per tile decides its commits."""
        return self.gathering and self.gather_invariant and self._plain_commit(self.resolved_mode())

    def render_plain_test(self, tid: str = "threadIdx.x") -> str:
        check = "true" if self.check else "false"
        return f"{self.loader}.template all_plain<{check}>({tid}, xp_{self.dst_name})"

    def _plain_commit(self, mode: str) -> bool:
        """The commit tests for plain divisors (vectorised gather loaders)."""
        return self.plain_apply_lambda is not None and self.plain_predicate is not None and mode in ("colvec", "rowvec")

    def _has_transform(self) -> bool:
        return self.transform_lambda is not None or self.value_transform is not None

    def stage_ptr(self, stage: str) -> str:
        if self.stages > 1:
            return f"&{self.dst_name}[{stage}][0][0]"
        return f"&{self.dst_name}[0][0]"

    def render_commit(self, stage: str = "0", tid: str = "threadIdx.x", plain: bool | None = None) -> str:
        """The commit to LDS stage ``stage``.  A loader with a plain chain
        tests its divisors at each commit (``plain`` None), or takes the
        plain (True) or the full chain (False) as its caller decided."""
        if self.is_dma:
            return ""
        if self.gathering:
            check = "true" if self.check else "false"
            d = self.dst_name
            if self._plain_commit(self.resolved_mode()):
                if plain is None:
                    return (
                        f"{self.loader}.template commit_apply_fast<{self.pitch}, {check}>"
                        f"({self.stage_ptr(stage)}, {tid}, xa_{d}, xq_{d}, xp_{d});"
                    )
                lam = f"xq_{d}" if plain else f"xa_{d}"
                return f"{self.loader}.template commit_apply<{self.pitch}, {check}>({self.stage_ptr(stage)}, {tid}, {lam});"
            return (
                f"{self.loader}.template commit_apply<{self.pitch}, {check}>"
                f"({self.stage_ptr(stage)}, {tid}, xa_{d});"
            )
        if self.defer_transform and self._has_transform() and self.resolved_mode() != "colvec_safe":
            check = "true" if self.check else "false"
            return (
                f"{self.loader}.template commit_xf<{self.pitch}, {check}>"
                f"({self.stage_ptr(stage)}, {tid}, {self.xform});"
            )
        return f"{self.loader}.template commit<{self.pitch}>({self.stage_ptr(stage)}, {tid});"

    def render(self, ctx: CodegenContext) -> str:
        tid = flat_tid(ctx)
        if self.is_dma:
            body = [self.render_decl(), self.render_fetch(tid, "0"), "__builtin_amdgcn_s_waitcnt(0);"]
        else:
            body = [self.render_decl(), self.render_fetch(tid), self.render_commit("0", tid)]
        return "{\n" + "\n".join(body) + "\n}"

    @property
    def lds_shape(self) -> tuple[int, ...]:
        """Shape of the LDS region written: the padded rows when the pitch is
        given, else the logical tile (the declaration's padding, if any, is
        not known here)."""
        rows, cols = self.tile_shape
        width = self.dst_pitch if self.dst_pitch is not None else cols
        return (self.stages, rows, width) if self.stages > 1 else (rows, width)

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        shape = self.lds_shape
        n = 1
        for d in shape:
            n *= d
        return (TgmemAccess(self.dst_name, "write", n, shape),)


@dataclass(frozen=True)
class TgStoreFragment:
    """LDS tile -> global (reference: memory.py:478-517), one element per
    lane per step, bounds-masked when limits are given."""

    name: str
    src_name: str
    dst_name: str
    dst_row_stride: str
    row_start: str
    col_start: str
    tile_shape: tuple[int, int]
    num_threads: int
    row_limit: str | None = None
    col_limit: str | None = None
    dst_col_stride: str = "1"
    kind: str = "store"

    def render(self, ctx: CodegenContext) -> str:
        rows, cols = self.tile_shape
        col_term = "gc" if self.dst_col_stride == "1" else f"(size_t)gc * {self.dst_col_stride}"
        store = f"{self.dst_name}[(size_t)gr * {self.dst_row_stride} + {col_term}] = {self.src_name}[r][c];"
        if self.row_limit is not None and self.col_limit is not None:
            store = f"if (gr < ({self.row_limit}) && gc < ({self.col_limit})) {{ {store} }}"
        return "\n".join(
            [
                f"for (unsigned idx = {flat_tid(ctx)}; idx < {rows * cols}u; idx += {self.num_threads}u) {{",
                f"    const unsigned r = idx / {cols}u, c = idx % {cols}u;",
                f"    const unsigned gr = ({self.row_start}) + r, gc = ({self.col_start}) + c;",
                f"    {store}",
                "}",
            ]
        )

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        rows, cols = self.tile_shape
        return (TgmemAccess(self.src_name, "read", rows * cols, self.tile_shape),)
