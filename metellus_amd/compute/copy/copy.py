"""Strided copy: the fallback for reshapes that cannot be views
(reference: src/compute/copy/copy.py:25-54).

Output position ``i`` (row-major) holds the source's logical element
``(i // cols, i % cols)``, read through the source strides, which are baked
in as literals (kernels are generated per shape).  Exact by construction:
pure data movement.  A source that iterates linearly (``Tensor.linear_step``
not None) never gets here -- its reshapes are views -- so the sources are
transposed views and other irregular strides.  Two forms:

* ``transpose`` -- a column-major source (row stride 1, column stride
  ``ld``), i.e. a transposed view: tiles staged through LDS, read along the
  source's contiguous axis and written along the output's, both coalesced;
  128-bit nontemporal loads and device-scope stores when the sizes and
  ``ld`` are multiples of 4, one element per lane otherwise.  Measured on
  MI355X, a transposed 4096x4096 view (64 MiB each way): 79.3 us with one
  lane per output element gathering through the strides, 35.1 us with
  scalar 64x64 tiles, 28.7 us with 128-bit 64x64 tiles and ordinary loads
  and stores, 24.2 us with the streaming policy, 23.7 us (5.66 TB/s) with
  128x64 tiles on 256 lanes, 23.6 us (5.69 TB/s) on 512 lanes (24.1 on 1024);
  64x128, 128x128 (256-1024 lanes), 256x64 and 64x256 tiles took 24.1-34.5 us.  Two forms with 4 x 4 blocks transposed
  in registers (four 128-bit loads of 4 consecutive j per lane) were slower,
  exact both (same run, 30 launches each): stored straight from registers to
  4 output rows, no LDS (4 lanes along i, so 64-byte reads): 25.4 us; staged
  through LDS with 128-bit writes and reads and an XOR swizzle (512-byte
  reads, 256-byte stores): 24.8-33.4 us over 7 tile shapes, against 24.0 for
  this form -- a lane's 4 consecutive source rows put the rows one load
  instruction touches 4 apart instead of adjacent;
* ``gather`` -- any other strides: one lane per output element, the
  unravel in 32-bit arithmetic when the element count allows.
"""

from __future__ import annotations

from dataclasses import dataclass

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess

# Transpose tile: TRANSPOSE_TILE_I elements along the source's contiguous
# axis (i, the output's row index) by TRANSPOSE_TILE_J along its strided
# axis (j, the output's contiguous one), TRANSPOSE_LANES lanes per workgroup.
TRANSPOSE_TILE_I = 128
TRANSPOSE_TILE_J = 64
TRANSPOSE_LANES = 512
TRANSPOSE_PAD = 1  # LDS row padding: column reads hit distinct banks
# Streaming cache policy of the 128-bit form: nontemporal loads and
# device-scope stores (written through L2), as the flat elementwise streams.
TRANSPOSE_STREAMING = True


def transpose_lds_shape(ti: int = 0, tj: int = 0) -> tuple[int, int]:
    """LDS tile of the transpose: one row per source column of the tile."""
    return (tj or TRANSPOSE_TILE_J, (ti or TRANSPOSE_TILE_I) + TRANSPOSE_PAD)


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
    tile_i: int = 64  # transpose: tile extent along the source's contiguous axis
    tile_j: int = 64  # ... and along its strided axis
    streaming: bool = False  # transpose: nontemporal loads, device-scope stores
    name: str = "strided_copy"
    kind: str = "compute"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        if self.mode == "transpose":
            shape = transpose_lds_shape(self.tile_i, self.tile_j)
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
        ti, tj, p = self.tile_i, self.tile_j, TRANSPOSE_PAD
        rows, cols, ld = self.input_rows, self.input_cols, self.input_col_stride
        lanes = ctx.tg_x
        head = [
            f"// source (i, j) at [i + j * {ld}]: tile i0..i0+{ti} x j0..j0+{tj}, staged as copy_tile[j][i]",
            f"const unsigned i0 = blockIdx.y * {ti}u, j0 = blockIdx.x * {tj}u;",
        ]
        if rows % 4 == 0 and cols % 4 == 0 and ld % 4 == 0:
            # 128-bit loads of 4 consecutive i and stores of 4 consecutive j
            # (a 4-float group is wholly inside or outside the matrix); the
            # transposed LDS reads (odd pitch) stay on distinct banks
            qi, qj = ti // 4, tj // 4
            if lanes % qi or lanes % qj or tj % (lanes // qi) or ti % (lanes // qj):
                raise ValueError(f"transpose tile {ti}x{tj} does not split over {lanes} lanes")
            ld4, st4 = ("mt_ld4_nt", "mt_st4_wt") if self.streaming else ("mt_ld4", "mt_st4")
            return "\n".join(
                [
                    *head,
                    f"const unsigned li = 4u * (threadIdx.x % {qi}u), lj = threadIdx.x / {qi}u;",
                    "#pragma unroll",
                    f"for (unsigned jj = lj; jj < {tj}u; jj += {lanes // qi}u) {{",
                    f"    const bool in = i0 + li < {rows}u && j0 + jj < {cols}u;",
                    f"    const mt_f32x4 v = in ? {ld4}("
                    f"{self.input_name} + (size_t)(j0 + jj) * {ld}u + i0 + li) : mt_f32x4{{0.f, 0.f, 0.f, 0.f}};",
                    "    copy_tile[jj][li] = v.x; copy_tile[jj][li + 1u] = v.y;",
                    "    copy_tile[jj][li + 2u] = v.z; copy_tile[jj][li + 3u] = v.w;",
                    "}",
                    "__syncthreads();",
                    f"const unsigned sj = 4u * (threadIdx.x % {qj}u), si = threadIdx.x / {qj}u;",
                    "#pragma unroll",
                    f"for (unsigned ii = si; ii < {ti}u; ii += {lanes // qj}u) {{",
                    f"    if (i0 + ii < {rows}u && j0 + sj < {cols}u)",
                    f"        {st4}({self.output_name} + (size_t)(i0 + ii) * {cols}u + j0 + sj, mt_f32x4{{",
                    "            copy_tile[sj][ii], copy_tile[sj + 1u][ii], copy_tile[sj + 2u][ii], copy_tile[sj + 3u][ii]});",
                    "}",
                ]
            ) + f"\n// LDS rows padded to {ti + p} floats"
        if lanes % ti or lanes % tj or tj % (lanes // ti) or ti % (lanes // tj):
            raise ValueError(f"transpose tile {ti}x{tj} does not split over {lanes} lanes")
        return "\n".join(
            [
                *head,
                f"const unsigned li = threadIdx.x % {ti}u, lj = threadIdx.x / {ti}u;",
                f"for (unsigned jj = lj; jj < {tj}u; jj += {lanes // ti}u) {{  // coalesced along i",
                "    const unsigned i = i0 + li, j = j0 + jj;",
                f"    copy_tile[jj][li] = (i < {rows}u && j < {cols}u) ? {self.input_name}[(size_t)j * {ld}u + i] : 0.f;",
                "}",
                "__syncthreads();",
                f"const unsigned sj = threadIdx.x % {tj}u, si = threadIdx.x / {tj}u;",
                f"for (unsigned ii = si; ii < {ti}u; ii += {lanes // tj}u) {{  // coalesced along j",
                "    const unsigned i = i0 + ii, j = j0 + sj;",
                f"    if (i < {rows}u && j < {cols}u) {self.output_name}[(size_t)i * {cols}u + j] = copy_tile[sj][ii];",
                "}",
            ]
        ) + f"\n// LDS rows padded to {ti + p} floats"
