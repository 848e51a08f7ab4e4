"""Reduction strategy: standalone, prologue-fused or epilogue-fused
last-axis reduction (reference: src/orchestrator/assembly/reduction.py:24-109).

Bindings ``(src, out, *extras)`` and dims ``(M, K)`` follow the reference.
The launch differs: 256-lane workgroups holding ``4/W`` rows with ``W``
waves per row (see ``compute.reduction.reduction``); grid ``(ceil(M/R), 1, 1)``.
"""

from __future__ import annotations

from metellus_amd.compute.fragments import CodegenContext, lds_decl
from metellus_amd.compute.reduction import reduction as _red
from metellus_amd.compute.reduction.reduction import (
    LastAxisReductionComputeFragment,
    LastAxisReductionSetupFragment,
    StoreReductionResultFragment,
    scratch_floats,
)
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.expressions import (
    build_reduction_epilogue_transform,
    chain_value_transform,
)
from metellus_amd.orchestrator.assembly.extras import Extras, input_param, output_param, param_name
from metellus_amd.orchestrator.ir import ReductionOp, Tensor
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel

WG_LANES = 256
FORCE_WAVES_PER_ROW: int | None = None  # tuning override


def reduction_waves_per_row(M: int, K: int) -> int:
    """Waves cooperating on one row: 1 when M rows already give >= 2048
    waves; otherwise up to 4, as long as each lane still gets >= 16 elements."""
    if FORCE_WAVES_PER_ROW is not None:
        return FORCE_WAVES_PER_ROW
    W = 1
    while W < 4 and M * W < 2048 and K >= 64 * (2 * W) * 16:
        W *= 2
    return W


def assemble_reduction(decision: DecisionView, function_name: str | None) -> KernelGroup:
    anchor = decision.anchor
    assert isinstance(anchor, ReductionOp)
    src = decision.prologue_a[0].operands[0] if decision.prologue_a else anchor.input
    assert isinstance(src, Tensor)
    M, K = src.shape
    final_out = decision.epilogue[-1].out if decision.epilogue else anchor.out
    extras = Extras(base_slots_by_key={src.buffer_key: 0, final_out.buffer_key: 1})
    helpers: list[str] = []
    prologue = None
    if decision.prologue_a:
        prologue = chain_value_transform(
            decision.prologue_a, row_var="row", col_var="idx", extras=extras, base_slot=2, name="prologue"
        )
        helpers.append(prologue.helper)
    epilogue = None
    if decision.epilogue:
        epilogue = build_reduction_epilogue_transform(decision.epilogue, name="epilogue")
        helpers.append(epilogue.helper)

    W = reduction_waves_per_row(M, K)
    R = WG_LANES // (64 * W)
    vec = src.col_stride == 1 and K % 4 == 0 and src.row_stride % 4 == 0
    setup = LastAxisReductionSetupFragment(rows_dim="M", name="reduction_setup", waves_per_row=W, rows_per_group=R)
    compute = LastAxisReductionComputeFragment(
        op=anchor.op,
        input_name=param_name(src.buffer_key),
        scratch_name="scratch",
        reduce_dim="K",
        row_stride=str(src.row_stride),
        col_stride=str(src.col_stride),
        name="reduction_compute",
        tg_x=WG_LANES,
        value_transform=prologue,
        waves_per_row=W,
        rows_per_group=R,
        vectorized=vec,
        unroll=_red.UNROLL,
        nt_load=_red.NT_LOAD,
    )
    store = StoreReductionResultFragment(
        output_name=param_name(final_out.buffer_key),
        scratch_name="scratch",
        name="reduction_store",
        tg_x=WG_LANES,
        value_transform=epilogue,
        waves_per_row=W,
    )
    n_scratch = scratch_floats(W, R)
    ctx = CodegenContext(
        function_name=function_name or f"reduce_{anchor.out.name}_fused",
        buffers=(input_param(src.buffer_key), output_param(final_out.buffer_key), *extras.buffers),
        dims=("M", "K"),
        tg_x=WG_LANES,
        tg_y=1,
        threadgroup_decls=(lds_decl("scratch", (n_scratch,)),) if n_scratch else (),
        helpers=tuple(helpers),
    )
    return KernelGroup(
        kernel=Kernel(fragments=(setup, compute, store), ctx=ctx),
        bindings=(src.buffer_key, final_out.buffer_key, *extras.bindings),
        dims=(M, K),
        grid=((M + R - 1) // R, 1, 1),
        threads=(WG_LANES, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )


def reduction_order(group: KernelGroup) -> dict:
    """The combine-order parameters of a reduction kernel (for the CPU
    replay of its exact order): op, waves per row, vector path."""
    frag = next(f for f in group.kernel.fragments if isinstance(f, LastAxisReductionComputeFragment))
    return {"op": frag.op, "waves_per_row": frag.W, "vectorized": frag._vec(), "unroll": frag.unroll}
