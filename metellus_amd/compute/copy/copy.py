"""Strided copy: the fallback for reshapes that cannot be views
(reference: src/compute/copy/copy.py:25-54).

Output position ``i`` (row-major) holds the source's logical element
``(i // cols, i % cols)``, read through the source strides, which are baked
in as literals (kernels are generated per shape).  Exact by construction:
pure data movement.  A source that iterates linearly (``Tensor.linear_step``
not None) never gets here -- its reshapes are views -- so the sources are
transposed views and other irregular strides.  Two forms:

* ``transpose`` -- a column-major source (row stride 1, column stride
  ``ld``), i.e. a transposed view: 64x64 tiles staged through LDS, read
  along the source's contiguous axis and written along the output's, both
  coalesced; 128-bit loads and stores when the sizes and ``ld`` are
  multiples of 4, one element per lane otherwise.  Measured on MI355X, a
  transposed 4096x4096 view (64 MiB each way): 79.3 us with one lane per
  output element gathering through the strides, 35.1 us with scalar tiles,
  28.4 us with 128-bit tiles (4.7 TB/s);
* ``gather`` -- any other strides: one lane per output element, the
  unravel in 32-bit arithmetic when the element count allows.
"""

from __future__ import annotations

from dataclasses import dataclass

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess

TRANSPOSE_TILE = 64
TRANSPOSE_PAD = 1  # LDS row padding: column reads hit distinct banks


def copy_mode(rows: int, cols: int, row_stride: int, col_stride: int) -> str:
    """The copy form for a (rows, cols) source with these strides."""
    if row_stride == 1 and rows > 1 and cols > 1:
        return "transpose"
    return "gather"


@dataclass(frozen=True)
class StridedCopyFragment:
    input_name: str
    output_name: str
    input_row_stride: int
    input_col_stride: int
    input_cols: int
    input_rows: int = 0
    mode: str = "gather"
    name: str = "strided_copy"
    kind: str = "compute"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        if self.mode == "transpose":
            shape = (TRANSPOSE_TILE, TRANSPOSE_TILE + TRANSPOSE_PAD)
            return (TgmemAccess("copy_tile", "write", shape[0] * shape[1], shape),)
        return ()

    def render(self, ctx: CodegenContext) -> str:
        if self.mode == "transpose":
            return self._render_transpose(ctx)
        return self._render_gather(ctx)

    def _render_gather(self, ctx: CodegenContext) -> str:
        idx = "unsigned" if 0 < self.input_rows * self.input_cols < 2**31 else "size_t"
        return "\n".join(
            [
                f"const {idx} global_idx = ({idx})blockIdx.x * {ctx.tg_x}u + threadIdx.x;",
                "if (global_idx >= N) return;",
                f"const {idx} in_row = global_idx / {self.input_cols}u;",
                f"const {idx} in_col = global_idx % {self.input_cols}u;",
                f"{self.output_name}[global_idx] = {self.input_name}"
                f"[(size_t)in_row * {self.input_row_stride}u + (size_t)in_col * {self.input_col_stride}u];",
            ]
        )

    def _render_transpose(self, ctx: CodegenContext) -> str:
        t, p = TRANSPOSE_TILE, TRANSPOSE_PAD
        rows, cols, ld = self.input_rows, self.input_cols, self.input_col_stride
        lanes = ctx.tg_x
        assert lanes % t == 0, "the transpose needs whole 64-lane rows"
        if rows % 4 == 0 and cols % 4 == 0 and ld % 4 == 0:
            # 128-bit loads of 4 consecutive i and stores of 4 consecutive j
            # (a 4-float group is wholly inside or outside the matrix); the
            # transposed LDS reads (pitch 65) stay on distinct banks
            q, step = t // 4, lanes // (t // 4)
            return "\n".join(
                [
                    f"// source (i, j) at [i + j * {ld}]: tile j0..j0+{t} x i0..i0+{t}, 4 floats per lane",
                    f"const unsigned i0 = blockIdx.y * {t}u, j0 = blockIdx.x * {t}u;",
                    f"const unsigned l4 = 4u * (threadIdx.x % {q}u), lr = threadIdx.x / {q}u;",
                    f"for (unsigned jj = lr; jj < {t}u; jj += {step}u) {{",
                    f"    const bool in = i0 + l4 < {rows}u && j0 + jj < {cols}u;",
                    "    const mt_f32x4 v = in ? mt_ld4("
                    f"{self.input_name} + (size_t)(j0 + jj) * {ld}u + i0 + l4) : mt_f32x4{{0.f, 0.f, 0.f, 0.f}};",
                    "    copy_tile[jj][l4] = v.x; copy_tile[jj][l4 + 1u] = v.y;",
                    "    copy_tile[jj][l4 + 2u] = v.z; copy_tile[jj][l4 + 3u] = v.w;",
                    "}",
                    "__syncthreads();",
                    f"for (unsigned ii = lr; ii < {t}u; ii += {step}u) {{",
                    f"    if (i0 + ii < {rows}u && j0 + l4 < {cols}u)",
                    f"        mt_st4({self.output_name} + (size_t)(i0 + ii) * {cols}u + j0 + l4, mt_f32x4{{",
                    "            copy_tile[l4][ii], copy_tile[l4 + 1u][ii], copy_tile[l4 + 2u][ii], copy_tile[l4 + 3u][ii]});",
                    "}",
                ]
            ) + f"\n// LDS rows padded to {t + p} floats"
        return "\n".join(
            [
                f"// source (i, j) at [i + j * {ld}]: tile j0..j0+{t} x i0..i0+{t}",
                f"const unsigned i0 = blockIdx.y * {t}u, j0 = blockIdx.x * {t}u;",
                f"const unsigned li = threadIdx.x % {t}u, lr = threadIdx.x / {t}u;",
                f"for (unsigned jj = lr; jj < {t}u; jj += {lanes // t}u) {{  // coalesced along i",
                "    const unsigned i = i0 + li, j = j0 + jj;",
                f"    copy_tile[jj][li] = (i < {rows}u && j < {cols}u) ? {self.input_name}[(size_t)j * {ld}u + i] : 0.f;",
                "}",
                "__syncthreads();",
                f"for (unsigned ii = lr; ii < {t}u; ii += {lanes // t}u) {{  // coalesced along j",
                "    const unsigned i = i0 + ii, j = j0 + li;",
                f"    if (i < {rows}u && j < {cols}u) {self.output_name}[(size_t)i * {cols}u + j] = copy_tile[li][ii];",
                "}",
            ]
        ) + f"\n// LDS rows padded to {t + p} floats"
