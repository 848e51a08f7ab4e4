"""Strided copy: the fallback for reshapes that cannot be views
(reference: src/compute/copy/copy.py:25-54).

One lane per output element: output position ``i`` (row-major) is unravelled
into the source's logical (row, col) and read through the source strides,
which are baked in as literals (kernels are generated per shape).  Exact by
construction: pure data movement."""

from __future__ import annotations

from dataclasses import dataclass

from metellus_amd.compute.fragments import CodegenContext, TgmemAccess


@dataclass(frozen=True)
class StridedCopyFragment:
    input_name: str
    output_name: str
    input_row_stride: int
    input_col_stride: int
    input_cols: int
    name: str = "strided_copy"
    kind: str = "compute"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()

    def render(self, ctx: CodegenContext) -> str:
        return "\n".join(
            [
                f"const size_t global_idx = (size_t)blockIdx.x * {ctx.tg_x}u + threadIdx.x;",
                "if (global_idx >= N) return;",
                f"const size_t in_row = global_idx / {self.input_cols}u;",
                f"const size_t in_col = global_idx % {self.input_cols}u;",
                f"{self.output_name}[global_idx] = {self.input_name}"
                f"[in_row * {self.input_row_stride}u + in_col * {self.input_col_stride}u];",
            ]
        )
