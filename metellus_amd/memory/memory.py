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
  padded row pitch.

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


def _is_int(s: str) -> bool:
    try:
        int(s)
    except (TypeError, ValueError):
        return False
    return True


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
    mode: str | None = None  # "colvec" | "rowvec" | "scalar" (default: from strides)
    transform_lambda: str | None = None
    # Apply the transform when the registers are written to LDS rather than
    # when the loads return, so a pipelined mainloop does not wait for the
    # next chunk's loads before its MFMAs.  Worth it when the transform reads
    # only small broadcast operands (those loads then happen at commit).
    defer_transform: bool = False

    @property
    def pitch(self) -> int:
        return self.dst_pitch if self.dst_pitch is not None else self.tile_shape[1]

    @property
    def check(self) -> bool:
        return self.row_limit is not None or self.col_limit is not None

    def resolved_mode(self) -> str:
        if self.mode is not None:
            return self.mode
        rows, cols = self.tile_shape
        rs, cs = self.src_row_stride, self.src_col_stride
        if cs == "1" and cols % 4 == 0 and self.pitch % 4 == 0 and (not _is_int(rs) or int(rs) % 4 == 0):
            return "colvec"
        if rs == "1" and rows % 4 == 0 and _is_int(cs) and int(cs) % 4 == 0:
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

    def render_decl(self) -> str:
        rows, cols = self.tile_shape
        tmpl = {"colvec": "mt_tile_colvec", "rowvec": "mt_tile_rowvec", "scalar": "mt_tile_scalar"}[self.resolved_mode()]
        return f"{tmpl}<{rows}, {cols}, {self.num_threads}> {self.loader};\nconst auto {self.xform} = {self._lambda()};"

    def render_fetch(self) -> str:
        rlim = self.row_limit if self.row_limit is not None else "0xffffffffu"
        clim = self.col_limit if self.col_limit is not None else "0xffffffffu"
        check = "true" if self.check else "false"
        mode = self.resolved_mode()
        deferred = self.defer_transform and self._has_transform()
        verb = "fetch_raw" if deferred else "fetch"
        head = f"{self.loader}.template {verb}<{check}>({self.src_name}, "
        if mode == "colvec":
            strides = f"{self.src_row_stride}"
        elif mode == "rowvec":
            strides = f"{self.src_col_stride}"
        else:
            strides = f"{self.src_row_stride}, {self.src_col_stride}"
        tail = ")" if deferred else f", {self.xform})"
        return f"{head}{strides}, {self.row_start}, {self.col_start}, {rlim}, {clim}, threadIdx.x{tail};"

    def _has_transform(self) -> bool:
        return self.transform_lambda is not None or self.value_transform is not None

    def stage_ptr(self, stage: str) -> str:
        if self.stages > 1:
            return f"&{self.dst_name}[{stage}][0][0]"
        return f"&{self.dst_name}[0][0]"

    def render_commit(self, stage: str = "0") -> str:
        if self.defer_transform and self._has_transform():
            check = "true" if self.check else "false"
            return (
                f"{self.loader}.template commit_xf<{self.pitch}, {check}>"
                f"({self.stage_ptr(stage)}, threadIdx.x, {self.xform});"
            )
        return f"{self.loader}.template commit<{self.pitch}>({self.stage_ptr(stage)}, threadIdx.x);"

    def render(self, ctx: CodegenContext) -> str:
        return "{\n" + "\n".join([self.render_decl(), self.render_fetch(), self.render_commit("0")]) + "\n}"

    @property
    def lds_shape(self) -> tuple[int, ...]:
        rows = self.tile_shape[0]
        return (self.stages, rows, self.pitch) if self.stages > 1 else (rows, self.pitch)

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
                f"for (unsigned idx = threadIdx.x; idx < {rows * cols}u; idx += {self.num_threads}u) {{",
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
