"""Matmul strategy: standalone, prologue-fused, tile- or register-epilogue
matmul (reference: src/orchestrator/assembly/matmul.py:33-285).

Kept from the reference: the strategy labels, the bindings (deduplicated
device inputs A/B, then the final output, then extra operands in order of
first use), dims ``(M, K, N)``, grid ``(N tiles, M tiles, 1)``, operand
strides read from the ``Tensor`` metadata (transposed views load
transposed; K^T is read along K with 128-bit loads, no transpose kernel).

gfx950 kernel: fp32 MFMA mainloop over double-buffered LDS, every epilogue
applied to the accumulator registers (both ``MATMUL_EPILOGUE_REGISTER`` and
``MATMUL_EPILOGUE_TG``; the label records the reference's decision), then a
direct store.  LDS holds only the A and B chunks.  When the output tiles
outnumber the workgroups resident at once, the grid is instead
``(P, 1, 1)`` workgroups looping over tiles (``PersistentTiles``); when
the tiles are not a whole number of rounds, the last round is split by
k-chunks (stream-K) through a workspace the runtime passes as the last
kernel parameter.
"""

from __future__ import annotations

import dataclasses

from metellus_amd.compute.fragments import BarrierFragment, CodegenContext, lds_decl
from metellus_amd.compute.matmul.config import (
    NUM_CUS,
    STREAM_K_MAX_WORKGROUPS,
    TileConfig,
    ceil_div,
    grid_for,
    is_aligned_shape,
    persistent_workgroups,
    resident_workgroups,
    select_tile_config,
    uses_stream_k,
)
from metellus_amd.compute.matmul.matmul import (
    MatmulComputeFragment,
    MatmulConfig,
    MatmulEpilogueStoreFragment,
    MatmulKResidentFragment,
    MatmulMainloopFragment,
    MatmulRowReduceFinishFragment,
    MatmulRowReduceSetupFragment,
    MatmulRowReduceStoreFragment,
    MatmulRowWavesFragment,
    MatmulSetupFragment,
    MatmulTileMappingFragment,
    PersistentLoopEndFragment,
    PersistentTiles,
    StreamKFixupFragment,
    ThreadIndexFragment,
    rr_lds_shape,
    rr_row_blocks,
    rr_workspace_bytes,
    stream_k_workspace_bytes,
)
from metellus_amd.memory.memory import TgLoadFragment, dma_offsets_fit
from metellus_amd.orchestrator.assembly.decision import DecisionView
from metellus_amd.orchestrator.assembly.expressions import ChainCode
from metellus_amd.orchestrator.assembly.extras import Extras, input_param, output_param, param_name
from metellus_amd.orchestrator.ir import MatmulOp, Tensor
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Kernel


def operand_load(
    *,
    name: str,
    src: Tensor,
    dst: str,
    tile: TileConfig,
    side: str,
    M: int,
    K: int,
    N: int,
    aligned: bool,
    k_limit: str = "K",
    prologue: ChainCode | None = None,
) -> TgLoadFragment:
    """Loader for the A (side "a": tile_M x tile_K at (tile_m0, k_chunk)) or
    B (side "b": tile_K x tile_N at (k_chunk, tile_n0)) operand."""
    rs, cs = src.row_stride, src.col_stride
    dma = None
    if side == "a" and tile.a_layout == "swz":
        dma = dict(src_row_stride=str(rs), row_start="tile_m0", col_start="k_chunk",
                   tile_shape=(tile.tile_M, tile.tile_K), dma_swizzle=True)
    elif side == "b" and tile.b_layout == "dense":
        dma = dict(src_row_stride=str(rs), row_start="k_chunk", col_start="tile_n0",
                   tile_shape=(tile.tile_K, tile.tile_N), dma_swizzle=False)
    elif side == "b" and tile.b_layout == "nswz":  # K^T-like view: rows of the source are B's columns
        dma = dict(src_row_stride=str(cs), row_start="tile_n0", col_start="k_chunk",
                   tile_shape=(tile.tile_N, tile.tile_K), dma_swizzle=True)
    if dma is not None:
        if prologue is not None or not aligned:
            raise ValueError(f"{name}: direct-to-LDS loads take no prologue and no bounds")
        return TgLoadFragment(name=name, src_name=param_name(src.buffer_key), dst_name=dst,
                              num_threads=tile.num_threads, dst_pitch=dma["tile_shape"][1],
                              stages=tile.stages, mode="dma", **dma)
    if side == "a":
        shape, pitch = (tile.tile_M, tile.tile_K), tile.lda
        row_start, col_start = "tile_m0", "k_chunk"
        row_lim, col_lim = "M", k_limit
        rows_total, cols_total = M, K
    else:
        shape, pitch = (tile.tile_K, tile.tile_N), tile.ldb
        row_start, col_start = "k_chunk", "tile_n0"
        row_lim, col_lim = k_limit, "N"
        rows_total, cols_total = K, N
    if cs == 1 and rs % 4 == 0 and cols_total % 4 == 0 and pitch % 4 == 0:
        mode = "colvec"
    elif rs == 1 and cs % 4 == 0 and rows_total % 4 == 0:
        mode = "rowvec"
    else:
        mode = "scalar"
    gather = gathers(prologue)
    lam = prologue.lambda_transform() if prologue is not None and not gather else None
    # one gather per 128-bit slot when the operands do not change along it
    along = {"colvec": "col", "rowvec": "row"}.get(mode)
    per_slot = gather and along is not None and along not in prologue.external_axes()
    # ... and when that vector axis is k (A along its columns, B along its
    # rows), a tile's k-chunks all need the same operands: gathered once per
    # tile (and a divisor's reciprocal becomes loop-invariant).  Measured on
    # MI355X, C5 O = (e / s1) @ V, bit-identical: 277.1 -> 272.1 us.
    invariant = per_slot and ((side == "a" and mode == "colvec") or (side == "b" and mode == "rowvec"))
    return TgLoadFragment(
        name=name,
        src_name=param_name(src.buffer_key),
        src_row_stride=str(rs),
        src_col_stride=str(cs),
        row_start=row_start,
        col_start=col_start,
        dst_name=dst,
        tile_shape=shape,
        num_threads=tile.num_threads,
        row_limit=None if aligned else row_lim,
        col_limit=None if aligned else col_lim,
        dst_pitch=pitch,
        stages=tile.stages,
        mode=mode,
        transform_lambda=lam,
        defer_transform=prologue is not None and not gather and prologue.broadcast_operands_only,
        gather_lambda=prologue.gather_lambda() if gather else None,
        apply_lambda=prologue.apply_lambda() if gather else None,
        plain_apply_lambda=prologue.plain_apply_lambda() if gather and PLAIN_COMMIT and prologue.plain_divisors() else None,
        plain_predicate=prologue.plain_predicate_lambda() if gather and PLAIN_COMMIT and prologue.plain_divisors() else None,
        n_gathered=len(prologue.externals) if gather else 0,
        gather_per_slot=per_slot,
        gather_invariant=invariant and GATHER_ONCE_PER_TILE,
    )


# Prologues load their external operands with the tile and apply the chain
# when the chunk is committed to LDS (gather / apply), so neither the chunk
# nor its operands are waited for before the current chunk's MFMAs and the
# commit issues no loads.  With full-size operands and a B chunk that also
# goes through registers, the k-chunks are GATHER_TILE_K wide so the extra
# registers fit beside a 256x256 tile's accumulators (broadcast operands
# cost one register per loader slot).
GATHER_PROLOGUES = True
GATHER_TILE_K = 16
GATHER_ONCE_PER_TILE = True  # k-invariant per-slot operands gathered with a tile's first chunk only
# Divisions inside matmul operand prologues use mt_div_fast (a refined
# reciprocal times the numerator, within 2 ulp of IEEE division); register
# epilogues and multi-anchor merges keep IEEE division.
FAST_DIV = True
# A gathering loader whose prologue divides only by gathered operands tests
# them (every lane, every in-bounds slot: 1 <= |y| < 2^125) and, when they
# pass, applies the chain with x * 1/y and no per-element branch -- the same
# bits as mt_div_fast.  Operands fixed for the tile (k-invariant gathers)
# are tested once per tile and the k loop runs in one of two versions;
# others are tested at each commit.  Measured on MI355X, C5 P @ V,
# bit-identical: 262.3 -> 259.9 us (-2.2 % in GRBM_GUI_ACTIVE cycles).
PLAIN_COMMIT = True


# Operand tiles with no prologue, a unit-stride axis and every chunk in bounds
# are loaded straight into LDS (global_load_lds_dwordx4): no prefetch
# registers and no LDS stores per chunk (measured on MI355X, results
# bit-identical: 4096^3 1001.6 -> 987.1 us; C5 S = Q @ K^T with K^T stored
# n-major 294.8 -> 289.4 us).
DMA_LOADS = True


def _dma_fits(rows: int, cols: int, threads: int) -> bool:
    slots = rows * cols // 4
    return cols % 4 == 0 and slots % 64 == 0 and (slots // 64) % (threads // 64) == 0


def dma_layouts(tile: TileConfig, srcs_a, srcs_b, pros_a, pros_b, aligned: bool) -> TileConfig:
    """``tile`` with the A / B tile layouts for direct-to-LDS loads where every
    operand of that side allows them: A row-major ("swz"); B row-major
    ("dense") or a transposed view read along K ("nswz")."""
    if not DMA_LOADS or not aligned or tile.stages != 2:
        return tile
    nt = tile.num_threads
    tm, tn, tk = tile.tile_M, tile.tile_N, tile.tile_K
    swz_k = tk in (16, 32)
    a_ok = (
        swz_k
        and all(p is None and t.col_stride == 1 and t.row_stride % 4 == 0 for t, p in zip(srcs_a, pros_a))
        and all(dma_offsets_fit(tm, tk, t.row_stride) for t in srcs_a)
        and _dma_fits(tm, tk, nt)
    )
    b_layout = "pad"
    if all(p is None for p in pros_b):
        if (
            all(t.col_stride == 1 and t.row_stride % 4 == 0 and dma_offsets_fit(tk, tn, t.row_stride) for t in srcs_b)
            and _dma_fits(tk, tn, nt)
        ):
            b_layout = "dense"
        elif (
            swz_k
            and all(t.row_stride == 1 and t.col_stride % 4 == 0 and dma_offsets_fit(tn, tk, t.col_stride) for t in srcs_b)
            and _dma_fits(tn, tk, nt)
        ):
            b_layout = "nswz"
    return dataclasses.replace(tile, a_layout="swz" if a_ok else "pad", b_layout=b_layout)


# 16-wave tiles (config.WIDE_TILES) for matmuls whose shape needs no bounds
# checks and whose prologues gather no full-size operands (or, with
# WIDE_GATHER_TILES, also for those).
WIDE_TILES = True
WIDE_GATHER_TILES = False

# Matmuls whose prologue gathers full-size operands issue the next k-chunk's
# register-path loads in LOAD_SPREAD parts spread over the current chunk's
# MFMAs (MatmulMainloopFragment.spread) instead of in one burst before them:
# a burst of 12 128-bit loads per lane held every wave in load issue while
# its MFMAs waited.  Measured on MI355X, C4 (h1*s*h2) @ W3, bit-identical
# outputs: 2881 -> 2790 us (2 parts) -> 2705 us (4 parts); spreading the
# direct-to-LDS B loads as well: 2738 us.  Kernels whose loads are all
# direct-to-LDS, or whose prologue reads only broadcast operands, were
# slower spread (4096^3 974 -> 996 / 1109 us, C4 X @ W1 2629 -> 2667 /
# 2728 us, C5 P @ V 276 -> 285 us), so they keep the burst.
LOAD_SPREAD = 4
LOAD_SPREAD_DMA = False  # spread direct-to-LDS loads too (measurements only)


# Each chunk's last group of 4 k-steps carried over the barrier into the next
# chunk (MatmulMainloopFragment.held) for mainloops of at least HELD_MIN_CHUNKS
# chunks whose loads are not spread.  Measured on MI355X as shader-clock
# cycles summed over the XCDs (GRBM_GUI_ACTIVE), bit-identical outputs:
# 4096^3 -1.0 %, C4 X @ W1 -0.6 %, C5 P @ V -0.5 to -0.8 %; C5 Q @ K^T
# (4 chunks) +3.0 % and C4 (h1*s*h2) @ W3 (spread loads, 236 VGPRs)
# +8.6 %, which keep the plain mainloop.
HELD_GROUPS = True
HELD_MIN_CHUNKS = 16


def held_groups(K: int, tile: TileConfig, spread: int) -> bool:
    return HELD_GROUPS and not spread and tile.tile_K >= 16 and K >= HELD_MIN_CHUNKS * tile.tile_K


# Matmuls 128 columns wide (C5 P @ V) on row-owning waves
# (MatmulRowWavesFragment): every wave owns 16 rows x 128 columns, so its A
# rows go from global memory straight into its registers and only B is
# staged in LDS, which leaves room for 64-wide k-chunks -- half the barriers
# of the LDS-tiled kernel, whose 256 x 128 tiles give each wave only 32
# MFMAs per 32-wide chunk.  Measured on MI355X, C5 P @ V (32 heads batched),
# same run: 249.8 -> 253.1 us against 257.6 -> 261.5 us for the LDS-tiled
# kernel (0.863-0.874 of the fp32 MFMA peak against 0.835-0.848); outputs
# agree to rounding (another MFMA shape: 16x16x4 instead of 32x32x2).
ROW_WAVES = True
ROW_WAVES_MIN_K = 1024


def row_waves(M: int, K: int, N: int, src_a: Tensor, src_b: Tensor, pro_a: ChainCode | None,
              pro_b: ChainCode | None, reduction) -> bool:
    """Whether a matmul takes the row-owning-wave kernel: 128 columns, whole
    256-row tiles, whole pairs of 64-wide chunks and at least
    ROW_WAVES_MIN_K of them, both operands read along rows with 16-byte
    aligned rows, no B prologue, an A prologue whose operands are fixed per
    row (or none), and no reduction epilogue."""
    if not ROW_WAVES or reduction is not None or pro_b is not None:
        return False
    if N != 128 or M % 256 or K % 128 or K < ROW_WAVES_MIN_K:
        return False
    if src_a.col_stride != 1 or src_a.row_stride % 4 or src_b.col_stride != 1 or src_b.row_stride % 4:
        return False
    if not dma_offsets_fit(64, 128, src_b.row_stride):
        return False
    return pro_a is None or pro_a.external_axes() <= {"row"}


# K-resident row waves (MatmulKResidentFragment): a matmul with K = 64 or
# 128 and an n-major B (attention's S = Q @ K^T reads K^T along K) keeps each
# wave's 16 rows of A for the whole K in registers and streams B through LDS
# in 128-column chunks; each chunk is a whole output tile, so no tile drains
# and the output stores of one chunk drain during the next chunk's MFMAs.
# The LDS-tiled kernel walks 256 x 256 tiles of only 4 (K = 128) k-chunks,
# and its 256 KiB of stores per tile ran after its MFMAs, not beside them.
K_RESIDENT = True
K_RESIDENT_MIN_N = 512
_RR_OP_NAMES = ("sum", "max", "min", "product")


def k_resident(M: int, K: int, N: int, src_a: Tensor, src_b: Tensor, pro_a: ChainCode | None,
               pro_b: ChainCode | None, reduction) -> bool:
    """Whether a matmul takes the K-resident row-wave kernel: K of 64 or 128,
    whole 256-row blocks, at least K_RESIDENT_MIN_N columns in whole
    128-column chunks, an output below 2 GiB, A read along rows and B along
    K (n-major), both with
    16-byte aligned rows, no B prologue, and an A prologue whose operands
    are fixed per row (or none).  A row-reduction epilogue (the matmul ->
    reduction extension) is computed in the same kernel.  The choice does
    not depend on the batch size, so a batched program sums in the same
    order as the same program alone."""
    if not K_RESIDENT or pro_b is not None:
        return False
    if reduction is not None and reduction.op not in _RR_OP_NAMES:
        return False
    if K not in (64, 128) or M % 256 or N % 128 or N < K_RESIDENT_MIN_N:
        return False
    if M * N * 4 >= 2**31:  # the stores address the output by 32-bit byte offsets
        return False
    strides = (src_a.row_stride, src_a.col_stride, src_b.row_stride, src_b.col_stride)
    if not all(isinstance(x, int) for x in strides):
        return False
    if src_a.col_stride != 1 or src_a.row_stride % 4 or src_b.row_stride != 1 or src_b.col_stride % 4:
        return False
    if not dma_offsets_fit(128, K, src_b.col_stride):
        return False
    return pro_a is None or pro_a.external_axes() <= {"row"}


def k_resident_chunks(M: int, N: int, batch: int = 1) -> int:
    """128-column chunks each workgroup of the K-resident kernel walks: as
    many as possible while the grid still gives every compute unit a
    workgroup -- the columns split into the fewest equal groups (a divisor
    of the chunk count) that fill NUM_CUS with the batch's row blocks.  The
    split does not change any sum's order."""
    total = N // 128
    want = ceil_div(NUM_CUS, batch * (M // 256))
    groups = next((d for d in range(1, total + 1) if total % d == 0 and d >= want), total)
    return total // groups


# One-tile-per-workgroup matmuls whose row tiles split evenly over the 8
# XCDs take the XCD-grouped tile order (MatmulTileMappingFragment.xcd_rows).
XCD_TILE_ORDER = False


def xcd_rows(grid: tuple[int, int, int]) -> int:
    """Row tiles per XCD of the XCD-grouped order for this grid (0: the
    plain order)."""
    gx, gy, _ = grid
    if not XCD_TILE_ORDER or gy % 8 or gx < 2:
        return 0
    return gy // 8


def load_spread(*prologues: ChainCode | None) -> int:
    """Spread parts for a mainloop whose A / B prologues are ``prologues``."""
    return LOAD_SPREAD if any(gathers_full_operands(p) for p in prologues) else 0


def gathers(prologue: ChainCode | None) -> bool:
    return GATHER_PROLOGUES and prologue is not None and len(prologue.externals) > 0


def gathers_full_operands(prologue: ChainCode | None) -> bool:
    return gathers(prologue) and not prologue.broadcast_operands_only


def b_tile_for(tile: TileConfig, src_b: Tensor, K: int, N: int) -> TileConfig:
    """Row pitch of the B tile in LDS.  A B operand read 128-bit along
    columns is committed with 128-bit stores and keeps a pitch that is a
    multiple of 4 floats.  Any other B (a transposed view such as K^T, or
    odd strides) is committed by 32-bit stores walking down columns, where a
    pitch of tile_N + 4 puts rows 0, 4, 8, ... of a column on colliding
    banks; an odd pitch (tile_N + 3) spreads them (measured on MI355X for
    the attention S = Q @ K^T kernel: 372.8 -> 360.5 us)."""
    if src_b.col_stride == 1 and src_b.row_stride % 4 == 0 and N % 4 == 0:
        return tile
    return dataclasses.replace(tile, b_pad=3)


def rr_local(M: int, N: int, tile: TileConfig, batch: int = 1) -> bool:
    """The row-reduction epilogue completes rows inside one workgroup (row
    blocks walked whole, ``PersistentTiles.row_blocks``) when a tile spans
    the whole row, or when the row blocks fill at least one round of the
    GPU's resident workgroups.  Otherwise (few, long rows) every tile runs
    in parallel and the row blocks are combined across workgroups through
    the workspace (an agent-scope release per tile: slower per tile, but
    not limited to a few workgroups)."""
    if ceil_div(N, tile.tile_N) == 1:
        return True
    return batch * ceil_div(M, tile.tile_M) >= NUM_CUS * rr_resident_workgroups(tile)


def rr_resident_workgroups(tile: TileConfig) -> int:
    """Resident workgroups of a matmul with the row-reduction epilogue: its
    per-wave-column row array sits in LDS beside the operand tiles."""
    rows, cols = rr_lds_shape(tile)
    return resident_workgroups(tile, extra_lds=4 * rows * cols)


def assemble_matmul(decision: DecisionView, function_name: str | None, batch: int = 1) -> KernelGroup:
    anchor = decision.anchor
    assert isinstance(anchor, MatmulOp)
    src_a = decision.prologue_a[0].operands[0] if decision.prologue_a else anchor.a
    src_b = decision.prologue_b[0].operands[0] if decision.prologue_b else anchor.b
    assert isinstance(src_a, Tensor) and isinstance(src_b, Tensor)
    M, K = anchor.a.shape
    N = anchor.b.shape[1]
    final_out = decision.epilogue[-1].out if decision.epilogue else anchor.out
    out_key = final_out.buffer_key

    slots: dict[str, int] = {}
    for key in (src_a.buffer_key, src_b.buffer_key):
        slots.setdefault(key, len(slots))
    out_slot = len(slots)
    base = out_slot + 1
    extras = Extras(base_slots_by_key={**slots, out_key: out_slot})

    helpers: list[str] = []
    pro_a = pro_b = None
    if decision.prologue_a:
        pro_a = ChainCode(decision.prologue_a, (src_a.name,), "prologue_a", fast_div=FAST_DIV)
        pro_a.register_extras(extras, base)
        helpers += pro_a.helpers()
    if decision.prologue_b:
        pro_b = ChainCode(decision.prologue_b, (src_b.name,), "prologue_b", fast_div=FAST_DIV)
        pro_b.register_extras(extras, base)
        helpers += pro_b.helpers()
    value_expr = None
    if decision.epilogue:
        epi = ChainCode(decision.epilogue, (anchor.out.name,), "epilogue")  # IEEE division: the output
        epi.register_extras(extras, base)
        helpers.append(epi.helper())
        value_expr = epi.scalar_call(["{a0}"], "row", "col")

    if row_waves(M, K, N, src_a, src_b, pro_a, pro_b, decision.reduction):
        return _assemble_row_waves(decision, function_name, src_a, src_b, pro_a, value_expr, slots, out_key,
                                   extras, helpers, M, K, N)
    if k_resident(M, K, N, src_a, src_b, pro_a, pro_b, decision.reduction):
        return _assemble_k_resident(decision, function_name, src_a, src_b, pro_a, value_expr, slots, out_key,
                                    extras, helpers, M, K, N, batch)

    full_gather = gathers_full_operands(pro_a) or gathers_full_operands(pro_b)
    wide = WIDE_TILES and (not full_gather or WIDE_GATHER_TILES)
    tile = b_tile_for(select_tile_config(M, K, N, batch=batch, wide=wide), src_b, K, N)
    aligned = is_aligned_shape(M, K, N, tile)
    if tile.num_threads > 512 and not aligned:
        # 16-wave tiles only without bounds checks (their masks cost registers)
        tile = b_tile_for(select_tile_config(M, K, N, batch=batch), src_b, K, N)
        aligned = is_aligned_shape(M, K, N, tile)

    tile = dma_layouts(tile, (src_a,), (src_b,), (pro_a,), (pro_b,), aligned)
    if full_gather and tile.b_layout == "pad":
        # a B chunk loaded through registers leaves no room for full-size
        # gathered operands at 32-wide chunks; a directly loaded B does
        # (measured, C4 (h1*s*h2) @ W3: 2.93 ms with 16-wide chunks, 2.89 ms
        # with W3 loaded directly and 32-wide chunks)
        tile = dataclasses.replace(tile, tile_K=min(tile.tile_K, GATHER_TILE_K), a_layout="pad", b_layout="pad")
        aligned = is_aligned_shape(M, K, N, tile)
        tile = dma_layouts(tile, (src_a,), (src_b,), (pro_a,), (pro_b,), aligned)
    config = MatmulConfig(
        tile=tile,
        aligned=aligned,
        M_dim_var="M",
        K_dim_var="K",
        N_dim_var="N",
        a_buffer_name=param_name(src_a.buffer_key),
        b_buffer_name=param_name(src_b.buffer_key),
        c_buffer_name=param_name(out_key),
        a_tile_name="A_tile",
        b_tile_name="B_tile",
    )
    config.validate()
    a_load = operand_load(name="load_A_tile", src=src_a, dst="A_tile", tile=tile, side="a",
                          M=M, K=K, N=N, aligned=aligned, prologue=pro_a)
    b_load = operand_load(name="load_B_tile", src=src_b, dst="B_tile", tile=tile, side="b",
                          M=M, K=K, N=N, aligned=aligned, prologue=pro_b)
    n_persistent = persistent_workgroups(M, N, tile, batch)
    red = decision.reduction
    # the row-reduction epilogue needs each tile whole in one workgroup
    stream_k = red is None and uses_stream_k(M, K, N, tile, n_persistent, batch)
    local_rr = red is not None and rr_local(M, N, tile, batch)
    if local_rr:
        n_persistent = min(ceil_div(M, tile.tile_M), max(1, NUM_CUS * rr_resident_workgroups(tile) // batch))
    persistent = PersistentTiles(tile.tile_M, tile.tile_N, stream_k=stream_k, tile_K=tile.tile_K,
                                 row_blocks=local_rr) if n_persistent else None
    spread = load_spread(pro_a, pro_b)
    mainloop = MatmulMainloopFragment(
        tile_K=tile.tile_K,
        fragments=(a_load, b_load, BarrierFragment("inputs_ready"), MatmulComputeFragment(config),
                   BarrierFragment("compute_done")),
        K_dim_var="K",
        persistent=persistent is not None,
        spread=spread,
        spread_dma=LOAD_SPREAD_DMA,
        held=held_groups(K, tile, spread),
    )
    if red is None:
        store = MatmulEpilogueStoreFragment(config, value_expr=value_expr, check=not aligned)
    else:
        if not local_rr and rr_row_blocks(M, tile, batch) > STREAM_K_MAX_WORKGROUPS:
            raise ValueError(
                f"{red.out.name}: the row-reduction epilogue counts row blocks in the workspace's "
                f"{STREAM_K_MAX_WORKGROUPS} flag words; {rr_row_blocks(M, tile, batch)} needed"
            )
        store = MatmulRowReduceStoreFragment(config, op=red.op, red_name=param_name(red.out.buffer_key),
                                             value_expr=value_expr, check=not aligned, local=local_rr)
    fragments = (
        *((MatmulRowReduceSetupFragment(local=local_rr),) if red is not None else ()),
        MatmulTileMappingFragment(persistent, xcd_rows=xcd_rows(grid_for(M, N, tile)) if persistent is None else 0),
        ThreadIndexFragment(tile),
        MatmulSetupFragment(config),
        mainloop,
        *((StreamKFixupFragment(config),) if stream_k else ()),
        store,
        *((PersistentLoopEndFragment(),) if persistent else ()),
        *((MatmulRowReduceFinishFragment(store),) if red is not None and not local_rr else ()),
    )
    red_keys = (red.out.buffer_key,) if red is not None else ()
    decls = (lds_decl("A_tile", tile.a_tile_shape()), lds_decl("B_tile", tile.b_tile_shape()))
    if red is not None:
        workspace = 0 if local_rr else rr_workspace_bytes(M, N, tile, batch)
        decls += (lds_decl("row_red", rr_lds_shape(tile)),)
    else:
        workspace = stream_k_workspace_bytes(tile.tile_M, tile.tile_N, n_persistent) if stream_k else 0
    ctx = CodegenContext(
        function_name=function_name or f"matmul_{anchor.out.name}_fused",
        buffers=(*(input_param(k) for k in slots), output_param(out_key), *extras.buffers,
                 *(output_param(k) for k in red_keys)),
        dims=("M", "K", "N"),
        tg_x=tile.tg_x,
        tg_y=1,
        threadgroup_decls=decls,
        helpers=tuple(helpers),
        workspace_bytes=workspace,
        workspace_batched=red is not None,
    )
    return KernelGroup(
        kernel=Kernel(fragments=fragments, ctx=ctx),
        bindings=(*slots, out_key, *extras.bindings, *red_keys),
        dims=(M, K, N),
        grid=(n_persistent, 1, 1) if n_persistent else grid_for(M, N, tile),
        threads=(tile.tg_x, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )


def _assemble_row_waves(decision: DecisionView, function_name: str | None, src_a: Tensor, src_b: Tensor,
                        pro_a: ChainCode | None, value_expr: str | None, slots: dict[str, int], out_key: str,
                        extras: Extras, helpers: list[str], M: int, K: int, N: int) -> KernelGroup:
    """The matmul as one MatmulRowWavesFragment (``row_waves`` holds)."""
    prologue = None
    if pro_a is not None:
        if gathers(pro_a):
            plain = PLAIN_COMMIT and pro_a.plain_divisors()
            prologue = ("gather", pro_a.gather_lambda(), pro_a.apply_lambda(),
                        pro_a.plain_apply_lambda() if plain else None,
                        pro_a.plain_predicate_lambda() if plain else None)
        else:
            prologue = ("transform", pro_a.lambda_transform())
    frag = MatmulRowWavesFragment(
        a_name=param_name(src_a.buffer_key),
        b_name=param_name(src_b.buffer_key),
        c_name=param_name(out_key),
        a_row_stride=src_a.row_stride,
        b_row_stride=src_b.row_stride,
        prologue=prologue,
        value_expr=value_expr,
    )
    ctx = CodegenContext(
        function_name=function_name or f"matmul_{decision.anchor.out.name}_fused",
        buffers=(*(input_param(k) for k in slots), output_param(out_key), *extras.buffers),
        dims=("M", "K", "N"),
        tg_x=MatmulRowWavesFragment.THREADS,
        tg_y=1,
        threadgroup_decls=(lds_decl("B_tile", (2, MatmulRowWavesFragment.TILE_K, MatmulRowWavesFragment.TILE_N)),),
        helpers=tuple(helpers),
    )
    return KernelGroup(
        kernel=Kernel(fragments=(frag,), ctx=ctx),
        bindings=(*slots, out_key, *extras.bindings),
        dims=(M, K, N),
        grid=(1, M // MatmulRowWavesFragment.TILE_M, 1),
        threads=(MatmulRowWavesFragment.THREADS, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )


def _assemble_k_resident(decision: DecisionView, function_name: str | None, src_a: Tensor, src_b: Tensor,
                         pro_a: ChainCode | None, value_expr: str | None, slots: dict[str, int], out_key: str,
                         extras: Extras, helpers: list[str], M: int, K: int, N: int, batch: int) -> KernelGroup:
    """The matmul as one MatmulKResidentFragment (``k_resident`` holds)."""
    prologue = None
    if pro_a is not None:
        if gathers(pro_a):
            prologue = ("gather", pro_a.gather_lambda(), pro_a.apply_lambda())
        else:
            prologue = ("transform", pro_a.lambda_transform())
    red = decision.reduction
    # a row reduction completes inside the workgroup: it walks whole rows
    chunks = k_resident_chunks(M, N, batch) if red is None else N // 128
    red_keys = (red.out.buffer_key,) if red is not None else ()
    frag = MatmulKResidentFragment(
        a_name=param_name(src_a.buffer_key),
        b_name=param_name(src_b.buffer_key),
        c_name=param_name(out_key),
        a_row_stride=src_a.row_stride,
        b_col_stride=src_b.col_stride,
        K=K,
        chunks=chunks,
        prologue=prologue,
        value_expr=value_expr,
        reduction=(red.op, param_name(red.out.buffer_key)) if red is not None else None,
    )
    ctx = CodegenContext(
        function_name=function_name or f"matmul_{decision.anchor.out.name}_fused",
        buffers=(*(input_param(k) for k in slots), output_param(out_key), *extras.buffers,
                 *(output_param(k) for k in red_keys)),
        dims=("M", "K", "N"),
        tg_x=MatmulKResidentFragment.THREADS,
        tg_y=1,
        threadgroup_decls=(lds_decl("B_tile", (2, MatmulKResidentFragment.TILE_N, K)),),
        helpers=tuple(helpers),
    )
    return KernelGroup(
        kernel=Kernel(fragments=(frag,), ctx=ctx),
        bindings=(*slots, out_key, *extras.bindings, *red_keys),
        dims=(M, K, N),
        grid=(N // (MatmulKResidentFragment.TILE_N * chunks), M // MatmulKResidentFragment.TILE_M, 1),
        threads=(MatmulKResidentFragment.THREADS, 1, 1),
        ops=decision.ops,
        strategy=decision.strategy,
    )
