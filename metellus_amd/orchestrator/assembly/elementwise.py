"""Elementwise strategy: one op or a fused chain, no anchor (reference:
src/orchestrator/assembly/elementwise.py:17-128).

Bindings ``(primary, out, *extras)`` and dims ``(M, N)`` (a 1-D primary is
(M, 1)) follow the reference.  The kernel is the register-resident stream of
``compute.elementwise.stream`` (256 lanes, no LDS)."""

from __future__ import annotations

from metellus_amd.compute.elementwise.stream import (
    ElementwiseStreamFragment,
    choose_layout,
    grid_for_layout,
)
from metellus_amd.compute.fragments import CodegenContext
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.expressions import ChainCode
from metellus_amd.orchestrator.assembly.extras import Extras, input_param, output_param
from metellus_amd.orchestrator.ir import Tensor
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel


def assemble_elementwise(decision: DecisionView, function_name: str | None) -> KernelGroup:
    chain = decision.chain_only
    assert chain, "elementwise decision must carry a chain"
    primary = chain[0].operands[0]
    assert isinstance(primary, Tensor)
    M, N = (primary.shape[0], 1) if len(primary.shape) == 1 else primary.shape
    final_out = chain[-1].out
    extras = Extras(base_slots_by_key={primary.buffer_key: 0, final_out.buffer_key: 1})
    code = ChainCode(tuple(chain), (primary.name,), "chain")
    code.register_extras(extras, 2)
    layout = choose_layout(primary, code.externals, M, N)
    body = ElementwiseStreamFragment(code=code, primary=primary, out_key=final_out.buffer_key, layout=layout)
    ctx = CodegenContext(
        function_name=function_name or f"elementwise_{final_out.name}_fused",
        buffers=(input_param(primary.buffer_key), output_param(final_out.buffer_key), *extras.buffers),
        dims=("M", "N"),
        tg_x=layout.threads,
        tg_y=1,
        helpers=(code.helper(),),
    )
    return KernelGroup(
        kernel=Kernel(fragments=(body,), ctx=ctx),
        bindings=(primary.buffer_key, final_out.buffer_key, *extras.bindings),
        dims=(M, N),
        grid=grid_for_layout(layout, M, N),
        threads=(layout.threads, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )
