"""Hand-composed kernels in the style of the reference's fragment-level
benches (reference: tests/bench_init.py, tests/bench_reduction.py,
tests/bench_elementwise.py, tests/bench_matmul.py): fragments, a
``CodegenContext`` and a ``Kernel`` built directly, no fusion pipeline.
Imports use the reference's module names.  Buffer declarations and the
preamble are written in HIP where the reference writes MSL; LDS tiles are
declared ``__shared__ alignas(16) float``."""

from __future__ import annotations

from compute.elementwise import ElementwiseComputeFragment, elementwise_arity
from compute.fragments import BarrierFragment, CodegenContext
from compute.init import ArangeFragment, CopyFragment, FillFragment
from compute.matmul import (
    MatmulAccumToDevFragment,
    MatmulAccumToTgFragment,
    MatmulComputeFragment,
    MatmulConfig,
    MatmulMainloopFragment,
    MatmulSetupFragment,
    MatmulTgToDevFragment,
    MatmulTileMappingFragment,
    ThreadIndexFragment,
)
from compute.matmul.config import grid_for, is_aligned_shape, select_tile_config
from compute.reduction import (
    LastAxisReductionComputeFragment,
    LastAxisReductionSetupFragment,
    StoreReductionResultFragment,
)
from memory import TgLoadFragment, TgStoreFragment
from runtime import Kernel

TG_X = 256


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


# ---- init (reference: tests/bench_init.py:17-40) -----------------------------


def _init_ctx(function_name: str, buffers: tuple[str, ...]) -> CodegenContext:
    return CodegenContext(function_name=function_name, buffers=buffers, dims=("N",), tg_x=TG_X, tg_y=1)


def fill_kernel(value: float) -> Kernel:
    return Kernel(fragments=(FillFragment("Out", "N", value=value),),
                  ctx=_init_ctx("fill_kernel", ("float* __restrict__ Out",)))


def arange_kernel(start: float, step: float) -> Kernel:
    return Kernel(fragments=(ArangeFragment("Out", "N", start=start, step=step),),
                  ctx=_init_ctx("arange_kernel", ("float* __restrict__ Out",)))


def copy_kernel() -> Kernel:
    return Kernel(fragments=(CopyFragment("Out", "In", "N"),),
                  ctx=_init_ctx("copy_kernel", ("float* __restrict__ Out", "const float* __restrict__ In")))


def init_grid(n: int) -> tuple[int, int, int]:
    return (ceil_div(n, TG_X), 1, 1)


# ---- one-row-per-workgroup reduction (reference: tests/bench_reduction.py:37-60)


def reduction_kernel(op: str) -> Kernel:
    fragments = (
        LastAxisReductionSetupFragment("M", "single_setup"),
        LastAxisReductionComputeFragment(op, "X", "tg_reduce", "N", "N", "single_reduce", TG_X),
        StoreReductionResultFragment("Out", "tg_reduce", "single_store", TG_X),
    )
    ctx = CodegenContext(
        function_name="reduce_last_axis_kernel",
        buffers=("const float* __restrict__ X", "float* __restrict__ Out"),
        dims=("M", "N"),
        tg_x=TG_X,
        tg_y=1,
        threadgroup_decls=(f"__shared__ alignas(16) float tg_reduce[{(TG_X + 31) // 32}];",),
    )
    return Kernel(fragments=fragments, ctx=ctx)


# ---- single-op elementwise over 16x16 LDS tiles, 32x8 lanes
# (reference: tests/bench_elementwise.py:77-218)


def elementwise_kernel(op, M, N, y_shape=None, cond_shape=None, y_broadcast="none", cond_broadcast="none"):
    tile_M = tile_N = 16
    tg_x, tg_y = 32, 8
    tile = (tile_M, tile_N)
    nt = tg_x * tg_y
    n_in = elementwise_arity(op)
    frags = [TgLoadFragment("load_X_tile", "X", "N", f"tg.y * {tile_M}", f"tg.x * {tile_N}", "X_tile", tile, nt, "M", "N")]
    if n_in >= 2:
        frags.append(TgLoadFragment(
            "load_Y_tile", "Y", "Y_stride",
            "0" if y_broadcast in ("scalar", "row") else f"tg.y * {tile_M}",
            "0" if y_broadcast in ("scalar", "col") else f"tg.x * {tile_N}",
            "Y_tile", tile, nt, "Y_rows", "Y_cols"))
    if n_in == 3:
        frags.append(TgLoadFragment(
            "load_Cond_tile", "Cond", "C_stride",
            "0" if cond_broadcast in ("scalar", "row") else f"tg.y * {tile_M}",
            "0" if cond_broadcast in ("scalar", "col") else f"tg.x * {tile_N}",
            "Cond_tile", tile, nt, "C_rows", "C_cols"))
    frags += [
        BarrierFragment("inputs_ready"),
        ElementwiseComputeFragment(op, "Out_tile", "X_tile", tile, nt,
                                   "Y_tile" if n_in >= 2 else None, "Cond_tile" if n_in == 3 else None,
                                   y_broadcast, cond_broadcast),
        BarrierFragment("output_ready"),
        TgStoreFragment("store_Out_tile", "Out_tile", "Out", "N", f"tg.y * {tile_M}", f"tg.x * {tile_N}",
                        tile, nt, "M", "N"),
    ]
    buffers = ["const float* __restrict__ X"]
    dim_names, dim_values = ["M", "N"], [M, N]
    decls = [f"__shared__ alignas(16) float X_tile[{tile_M}][{tile_N}];"]
    bindings = ["X"]
    if n_in >= 2:
        buffers.append("const float* __restrict__ Y")
        dim_names += ["Y_rows", "Y_cols", "Y_stride"]
        dim_values += [y_shape[0], y_shape[1], y_shape[1]]
        decls.append(f"__shared__ alignas(16) float Y_tile[{tile_M}][{tile_N}];")
        bindings.append("Y")
    if n_in == 3:
        buffers.append("const float* __restrict__ Cond")
        dim_names += ["C_rows", "C_cols", "C_stride"]
        dim_values += [cond_shape[0], cond_shape[1], cond_shape[1]]
        decls.append(f"__shared__ alignas(16) float Cond_tile[{tile_M}][{tile_N}];")
        bindings.append("Cond")
    buffers.append("float* __restrict__ Out")
    bindings.append("Out")
    decls.append(f"__shared__ alignas(16) float Out_tile[{tile_M}][{tile_N}];")
    ctx = CodegenContext(
        function_name="elementwise_kernel",
        buffers=tuple(buffers),
        dims=tuple(dim_names),
        tg_x=tg_x,
        tg_y=tg_y,
        threadgroup_decls=tuple(decls),
        preamble=(
            "const uint2 tg = make_uint2(blockIdx.x, blockIdx.y);",
            f"const unsigned flat_tid = threadIdx.y * {tg_x}u + threadIdx.x;",
        ),
    )
    grid = (ceil_div(N, tile_N), ceil_div(M, tile_M), 1)
    return Kernel(fragments=tuple(frags), ctx=ctx), tuple(bindings), tuple(dim_values), grid, (tg_x, tg_y, 1)


# ---- GEMM from matmul fragments (reference: tests/bench_matmul.py:51-128) ----


def gemm_kernel(m: int, k: int, n: int):
    tile = select_tile_config(m, k, n)
    aligned = is_aligned_shape(m, k, n, tile)
    config = MatmulConfig(tile, aligned, "M", "K", "N", "A", "B", "C", "A_tile", "B_tile", "C_tile")
    row_limit = None if aligned else "M"
    k_limit = None if aligned else "K"
    n_limit = None if aligned else "N"
    c_tile_decl = () if aligned else (
        f"__shared__ alignas(16) float C_tile[{tile.tile_M}][{tile.tile_N + tile.c_pad}];",)
    fragments = (
        MatmulTileMappingFragment(),
        ThreadIndexFragment(tile),
        MatmulSetupFragment(config),
        MatmulMainloopFragment(
            tile_K=tile.tile_K,
            fragments=(
                TgLoadFragment(name="load_A_tile", src_name="A", src_row_stride="K",
                               row_start=f"tg.y * {tile.tile_M}", col_start="k_chunk", dst_name="A_tile",
                               tile_shape=(tile.tile_M, tile.tile_K), num_threads=tile.num_threads,
                               row_limit=row_limit, col_limit=k_limit),
                TgLoadFragment(name="load_B_tile", src_name="B", src_row_stride="N",
                               row_start="k_chunk", col_start=f"tg.x * {tile.tile_N}", dst_name="B_tile",
                               tile_shape=(tile.tile_K, tile.tile_N), num_threads=tile.num_threads,
                               row_limit=k_limit, col_limit=n_limit),
                BarrierFragment("inputs_ready"),
                MatmulComputeFragment(config),
                BarrierFragment("compute_done"),
            ),
            K_dim_var="K",
        ),
        *((MatmulAccumToDevFragment(config),) if aligned else
          (MatmulAccumToTgFragment(config), BarrierFragment("c_tile_ready"), MatmulTgToDevFragment(config))),
    )
    ctx = CodegenContext(
        function_name="matmul_kernel",
        buffers=("const float* __restrict__ A", "const float* __restrict__ B", "float* __restrict__ C"),
        dims=("M", "K", "N"),
        tg_x=tile.tg_x,
        tg_y=tile.tg_y,
        threadgroup_decls=(
            f"__shared__ alignas(16) float A_tile[{tile.tile_M}][{tile.tile_K + tile.a_pad}];",
            f"__shared__ alignas(16) float B_tile[{tile.tile_K}][{tile.tile_N + tile.b_pad}];",
            *c_tile_decl,
        ),
    )
    return Kernel(fragments=fragments, ctx=ctx), tile, aligned, grid_for(m, n, tile)


GEMM_SHAPES = [
    (512, 512, 512), (1024, 64, 1024), (16, 4096, 16), (17, 19, 23), (63, 31, 65), (64, 33, 64),
    (65, 64, 17), (127, 129, 131), (1, 1, 1), (3, 70, 5), (130, 7, 96), (4096, 512, 4096), (8192, 64, 8192),
]
UNARY_OPS = ["negate", "absolute", "exp", "log", "sqrt", "recip", "sin", "cos", "tanh", "floor", "ceil", "sign"]
BINARY_OPS = ["add", "subtract", "mul", "div", "max", "min", "pow", "equal", "not_equal", "lt", "gt", "ge", "le"]
