"""Shape (copy) strategy: strided gather into a fresh dense buffer
(reference: src/orchestrator/assembly/shape.py:14-68).  Bindings
``(in, out)``, dims ``(N,)``, 256 lanes per workgroup, one element per lane."""

from __future__ import annotations

from metellus_amd.compute.copy.copy import StridedCopyFragment
from metellus_amd.compute.fragments import CodegenContext
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.extras import input_param, output_param, param_name
from metellus_amd.orchestrator.ir import ShapeOp
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel

LANES = 256


def assemble_shape(decision: DecisionView, function_name: str | None) -> KernelGroup:
    op = decision.shape_op
    assert isinstance(op, ShapeOp)
    src, out = op.input, op.out
    n = out.element_count
    if len(src.shape) == 2:
        cols = src.shape[1]
    elif len(src.shape) == 1:
        cols = src.shape[0]
    else:
        raise ValueError(f"ShapeOp input must be 1D or 2D in v0; got shape {src.shape}")
    frag = StridedCopyFragment(
        input_name=param_name(src.buffer_key),
        output_name=param_name(out.buffer_key),
        input_row_stride=src.row_stride,
        input_col_stride=src.col_stride,
        input_cols=cols,
    )
    ctx = CodegenContext(
        function_name=function_name or f"shape_{out.name}",
        buffers=(input_param(src.buffer_key), output_param(out.buffer_key)),
        dims=("N",),
        tg_x=LANES,
        tg_y=1,
    )
    return KernelGroup(
        kernel=Kernel(fragments=(frag,), ctx=ctx),
        bindings=(src.buffer_key, out.buffer_key),
        dims=(n,),
        grid=((n + LANES - 1) // LANES, 1, 1),
        threads=(LANES, 1, 1),
        ops=(op,),
        strategy=decision.strategy,
    )
