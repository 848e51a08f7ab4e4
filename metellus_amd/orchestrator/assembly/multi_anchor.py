"""Multi-anchor strategy: two matmuls over the same (M, N) tile merged by one
binary elementwise op (reference: src/orchestrator/assembly/multi_anchor.py:50-355).

Kept from the reference: DIAMOND_SHARED vs MULTI_PRODUCER_CONVERGENT, the
deduplicated input bindings (A0, B0, [A1,] B1 in that order, then the
output, then prologue extras), dims ``(M, K, N)`` (shared) or
``(M, K0, K1, N)``, the tile chosen for the larger K.

gfx950 kernel: two register accumulator sets ``acc_0``/``acc_1``.  The
diamond runs one mainloop that loads the shared A chunk once and both B
chunks; otherwise two mainloops run back to back, and their LDS tiles have
disjoint lifetimes, so the aliasing pass gives A1/B1 the storage of A0/B0.
The merge op is applied per register and stored directly -- no C tiles.
The diamond takes the persistent tile loop (and stream-K for a partial last
round, handing over both accumulator sets) like a single matmul; the
two-mainloop form keeps one tile per workgroup.
"""

from __future__ import annotations

from metellus_amd.compute.fragments import BarrierFragment, CodegenContext, lds_decl
from metellus_amd.compute.matmul.config import (
    grid_for,
    is_aligned_shape,
    persistent_workgroups,
    select_tile_config,
    uses_stream_k,
)
from metellus_amd.compute.matmul.matmul import (
    MatmulComputeFragment,
    MatmulConfig,
    MatmulEpilogueStoreFragment,
    MatmulMainloopFragment,
    MatmulSetupFragment,
    MatmulTileMappingFragment,
    PersistentLoopEndFragment,
    PersistentTiles,
    StreamKFixupFragment,
    ThreadIndexFragment,
    stream_k_workspace_bytes,
)
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.expressions import ChainCode
from metellus_amd.orchestrator.assembly.extras import Extras, input_param, output_param, param_name
from metellus_amd.orchestrator.assembly import matmul as _mm
from metellus_amd.orchestrator.assembly.matmul import b_tile_for, dma_layouts, operand_load
from metellus_amd.orchestrator.ir import Tensor
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel


def assemble_multi_anchor(decision: DecisionView, function_name: str | None, batch: int = 1) -> KernelGroup:
    anchors = decision.anchors
    merge = decision.merge_elem
    assert anchors is not None and len(anchors) == 2 and merge is not None
    a0, a1 = anchors
    M, N = a0.out.shape
    assert a1.out.shape == (M, N), "multi-anchor: anchors must share output shape"
    K0, K1 = a0.a.shape[1], a1.a.shape[1]
    shared = decision.shared_a and K0 == K1
    pro_a = decision.prologues_a or ((), ())
    pro_b = decision.prologues_b or ((), ())
    src_a = tuple(pro_a[i][0].operands[0] if pro_a[i] else anchors[i].a for i in range(2))
    src_b = tuple(pro_b[i][0].operands[0] if pro_b[i] else anchors[i].b for i in range(2))
    assert all(isinstance(t, Tensor) for t in (*src_a, *src_b))
    out_key = merge.out.buffer_key
    tile = select_tile_config(M, max(K0, K1), N, anchors=2, batch=batch)
    padded = [b_tile_for(tile, src_b[i], (K0, K1)[i], N) for i in range(2)]
    if all(p.b_pad != tile.b_pad for p in padded):
        tile = padded[0]  # both B tiles committed by 32-bit stores
    aligned = is_aligned_shape(M, K0, N, tile) and is_aligned_shape(M, K1, N, tile)

    order = (src_a[0], src_b[0], src_b[1]) if shared else (src_a[0], src_b[0], src_a[1], src_b[1])
    keys: list[str] = []
    for t in order:
        if t.buffer_key not in keys:
            keys.append(t.buffer_key)
    out_slot = len(keys)
    base = out_slot + 1
    extras = Extras(base_slots_by_key={**{k: i for i, k in enumerate(keys)}, out_key: out_slot})

    helpers: list[str] = []

    def prologue(chain, src, label):
        if not chain:
            return None
        code = ChainCode(tuple(chain), (src.name,), label, fast_div=_mm.FAST_DIV)
        code.register_extras(extras, base)
        helpers.extend(code.helpers())
        return code

    tf_a = tuple(prologue(pro_a[i], src_a[i], f"prologue_a{i}") for i in range(2))
    tf_b = tuple(prologue(pro_b[i], src_b[i], f"prologue_b{i}") for i in range(2))
    merge_chain = decision.merge_chain or (merge,)
    merge_code = ChainCode(merge_chain, (a0.out.name, a1.out.name), "merge")  # IEEE division: the output
    if merge_code.externals:
        raise ValueError("multi-anchor: the merge reads tensors other than the two matmul outputs")
    helpers.append(merge_code.helper())
    value_expr = merge_code.call(["{a0}", "{a1}"], [])

    if shared:
        tile = dma_layouts(tile, (src_a[0],), src_b, (tf_a[0],), tf_b, aligned)
    kvars = ("K", "K") if shared else ("K0", "K1")
    ks = (K0, K1)
    configs = tuple(
        MatmulConfig(
            tile=tile,
            aligned=aligned,
            M_dim_var="M",
            K_dim_var=kvars[i],
            N_dim_var="N",
            a_buffer_name=param_name(src_a[i].buffer_key),
            b_buffer_name=param_name(src_b[i].buffer_key),
            c_buffer_name=param_name(out_key),
            a_tile_name="A_tile" if shared else f"A{i}_tile",
            b_tile_name=f"B{i}_tile",
        )
        for i in range(2)
    )
    configs[0].validate()
    suffixes = ("_0", "_1")

    def b_load(i):
        return operand_load(name=f"load_B{i}_tile", src=src_b[i], dst=f"B{i}_tile", tile=tile, side="b",
                            M=M, K=ks[i], N=N, aligned=aligned, k_limit=kvars[i], prologue=tf_b[i])

    n_persistent = persistent_workgroups(M, N, tile, batch, anchors=2) if shared else None
    stream_k = uses_stream_k(M, K0, N, tile, n_persistent, batch)
    persistent = PersistentTiles(tile.tile_M, tile.tile_N, stream_k=stream_k, tile_K=tile.tile_K) \
        if n_persistent else None
    if shared:
        a_load = operand_load(name="load_A_tile", src=src_a[0], dst="A_tile", tile=tile, side="a",
                              M=M, K=K0, N=N, aligned=aligned, k_limit="K")
        mainloops = [
            MatmulMainloopFragment(
                tile_K=tile.tile_K,
                fragments=(
                    a_load,
                    b_load(0),
                    b_load(1),
                    BarrierFragment("inputs_ready"),
                    MatmulComputeFragment(configs[0], accumulator_suffix=suffixes[0]),
                    MatmulComputeFragment(configs[1], accumulator_suffix=suffixes[1]),
                    BarrierFragment("compute_done"),
                ),
                K_dim_var="K",
                persistent=persistent is not None,
                spread=_mm.load_spread(*tf_b),
                spread_dma=_mm.LOAD_SPREAD_DMA,
            )
        ]
    else:
        mainloops = []
        for i in range(2):
            a_load = operand_load(name=f"load_A{i}_tile", src=src_a[i], dst=f"A{i}_tile", tile=tile, side="a",
                                  M=M, K=ks[i], N=N, aligned=aligned, k_limit=kvars[i], prologue=tf_a[i])
            mainloops.append(
                MatmulMainloopFragment(
                    tile_K=tile.tile_K,
                    fragments=(
                        a_load,
                        b_load(i),
                        BarrierFragment(f"inputs{i}_ready"),
                        MatmulComputeFragment(configs[i], accumulator_suffix=suffixes[i]),
                        BarrierFragment(f"compute{i}_done"),
                    ),
                    K_dim_var=kvars[i],
                    spread=_mm.load_spread(tf_a[i], tf_b[i]),
                    spread_dma=_mm.LOAD_SPREAD_DMA,
                )
            )

    store = MatmulEpilogueStoreFragment(configs[0], value_expr=value_expr, suffixes=suffixes, check=not aligned)
    fragments = (
        MatmulTileMappingFragment(persistent),
        ThreadIndexFragment(tile),
        MatmulSetupFragment(configs[0], accumulator_suffix=suffixes[0]),
        MatmulSetupFragment(configs[1], accumulator_suffix=suffixes[1], emit_thread_coords=False),
        *mainloops,
        *((StreamKFixupFragment(configs[0], suffixes=suffixes),) if stream_k else ()),
        store,
        *((PersistentLoopEndFragment(),) if persistent else ()),
    )
    decls = []
    if shared:
        decls.append(lds_decl("A_tile", tile.a_tile_shape()))
    else:
        decls += [lds_decl(f"A{i}_tile", tile.a_tile_shape()) for i in range(2)]
    decls += [lds_decl(f"B{i}_tile", tile.b_tile_shape()) for i in range(2)]
    if shared:
        dim_names, dim_values = ("M", "K", "N"), (M, K0, N)
    else:
        dim_names, dim_values = ("M", "K0", "K1", "N"), (M, K0, K1, N)
    ctx = CodegenContext(
        # the reference's name; a merge chain (an extension) is named apart
        function_name=function_name or (
            f"multi_anchor_{merge.out.name}_fused" if len(merge_chain) == 1 else f"multi_anchor_chain_{merge.out.name}_fused"
        ),
        buffers=(*(input_param(k) for k in keys), output_param(out_key), *extras.buffers),
        dims=dim_names,
        tg_x=tile.tg_x,
        tg_y=1,
        threadgroup_decls=tuple(decls),
        helpers=tuple(helpers),
        workspace_bytes=stream_k_workspace_bytes(tile.tile_M, tile.tile_N, n_persistent, anchors=2) if stream_k else 0,
    )
    return KernelGroup(
        kernel=Kernel(fragments=fragments, ctx=ctx),
        bindings=(*keys, out_key, *extras.bindings),
        dims=dim_values,
        grid=(n_persistent, 1, 1) if n_persistent else grid_for(M, N, tile),
        threads=(tile.tg_x, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )
