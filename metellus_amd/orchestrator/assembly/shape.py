"""Shape (copy) strategy: strided gather into a fresh dense buffer
(reference: src/orchestrator/assembly/shape.py:14-68).  Bindings
``(in, out)`` and dims ``(N,)`` as in the reference; 256 lanes per
workgroup.  The copy form follows the source layout
(``compute.copy.copy_mode``): LDS tiles for transposed views (grid over the
tiles, ``TRANSPOSE_TILE_I`` x ``TRANSPOSE_TILE_J``), one element per lane
otherwise."""

from __future__ import annotations

from metellus_amd.compute.copy import copy as cp
from metellus_amd.compute.copy.copy import StridedCopyFragment, copy_mode
from metellus_amd.compute.fragments import CodegenContext, lds_decl
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.extras import input_param, output_param, param_name
from metellus_amd.orchestrator.ir import ShapeOp
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel

LANES = 256


def _ceil(a: int, b: int) -> int:
    return (a + b - 1) // b


def assemble_shape(decision: DecisionView, function_name: str | None) -> KernelGroup:
    op = decision.shape_op
    assert isinstance(op, ShapeOp)
    src, out = op.input, op.out
    n = out.element_count
    if len(src.shape) == 2:
        rows, cols = src.shape
    elif len(src.shape) == 1:
        rows, cols = 1, src.shape[0]
    else:
        raise ValueError(f"ShapeOp input must be 1D or 2D in v0; got shape {src.shape}")
    mode = copy_mode(rows, cols, src.row_stride, src.col_stride)
    ti, tj = cp.TRANSPOSE_TILE_I, cp.TRANSPOSE_TILE_J
    lanes = cp.TRANSPOSE_LANES if mode == "transpose" else LANES
    frag = StridedCopyFragment(
        input_name=param_name(src.buffer_key),
        output_name=param_name(out.buffer_key),
        input_row_stride=src.row_stride,
        input_col_stride=src.col_stride,
        input_cols=cols,
        input_rows=rows,
        mode=mode,
        tile_i=ti,
        tile_j=tj,
        streaming=cp.TRANSPOSE_STREAMING,
    )
    if mode == "transpose":
        grid = (_ceil(cols, tj), _ceil(rows, ti), 1)
    else:
        grid = (_ceil(n, LANES), 1, 1)
    decls = (lds_decl("copy_tile", cp.transpose_lds_shape(ti, tj)),) if mode == "transpose" else ()
    ctx = CodegenContext(
        function_name=function_name or f"shape_{out.name}",
        buffers=(input_param(src.buffer_key), output_param(out.buffer_key)),
        dims=("N",),
        tg_x=lanes,
        tg_y=1,
        threadgroup_decls=decls,
    )
    return KernelGroup(
        kernel=Kernel(fragments=(frag,), ctx=ctx),
        bindings=(src.buffer_key, out.buffer_key),
        dims=(n,),
        grid=grid,
        threads=(lanes, 1, 1),
        ops=(op,),
        strategy=decision.strategy,
    )
