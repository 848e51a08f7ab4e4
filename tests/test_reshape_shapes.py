"""Views vs copies: transpose / reshape metadata, ShapeOp emission and the
strides the generated kernels use.  Restates the structural halves of the
reference's tests/test_reshape.py and tests/test_shape_transforms.py (the
MSL substrings retargeted to the HIP the gfx950 templates emit)."""

import pytest

from orchestrator import Operations, ShapeOp, Tensor
from orchestrator.assembly import assemble
from orchestrator.fusion import fuse
from orchestrator.kernel_group import FusionStrategy

from metellus_amd.runtime import hip_backend


def test_tensor_view_basics():
    assert Tensor("x", (8, 16)).buffer_key == "x"
    assert Tensor("x", (8, 16)).is_contiguous() and Tensor("v", (64,)).is_contiguous()
    assert not Tensor("x", (8, 16)).transpose("x_T").is_contiguous()
    v = Tensor("x", (8, 16)).reshape_view((128,), name="x_flat")
    assert (v.name, v.buffer_key, v.shape, v.row_stride, v.col_stride) == ("x_flat", "x", (128,), 1, 0)
    v = Tensor("x", (8, 16)).reshape_view((4, 32), name="x_r")
    assert (v.buffer_key, v.shape, v.row_stride, v.col_stride) == ("x", (4, 32), 32, 1)


def test_reshape_view_errors():
    t = Tensor("x", (8, 16)).transpose("x_T")
    with pytest.raises(ValueError, match="linearly-iterable"):
        t.reshape_view((128,), name="bad")
    with pytest.raises(ValueError):
        Tensor("x", (8, 16)).reshape_view((9, 16), name="bad")
    with pytest.raises(ValueError):
        Tensor("x", (8, 16)).reshape_view((2, 4, 16), name="bad")


def test_same_shape_reshape_keeps_strides():
    t = Tensor("x", (8, 16)).transpose("x_T")
    v = t.reshape_view((16, 8), name="v")
    assert v.buffer_key == "x" and (v.row_stride, v.col_stride) == (1, 16) and v.layout is t.layout


@pytest.mark.parametrize(
    "src,new", [((8, 16), (128,)), ((8, 16), (16, 8)), ((8, 16), (4, 32)), ((8, 16), (32, 4)), ((128,), (8, 16)), ((128,), (16, 8)), ((64,), (64,))]
)
def test_contiguous_reshape_is_view(src, new):
    ops = Operations()
    ops.input("X", shape=src)
    v = ops.reshape("X", new, out="Y")
    assert ops.build() == [] and v.buffer_key == "X" and v.shape == new


@pytest.mark.parametrize("src,new", [((8, 16), (8, 16)), ((1, 64), (64,)), ((64, 1), (64,))])
def test_degenerate_reshapes_are_views(src, new):
    ops = Operations()
    ops.input("X", shape=src)
    v = ops.reshape("X", new, out="Y")
    assert ops.build() == [] and v.buffer_key == "X"


@pytest.mark.parametrize(
    "shape,rs,cs,new,want",
    [
        ((12,), 3, 0, (4, 3), (9, 3)),
        ((12,), 3, 0, (3, 4), (12, 3)),
        ((12,), 3, 0, (2, 6), (18, 3)),
        ((12,), 3, 0, (12,), (3, 0)),
        ((1, 6), 0, 5, (2, 3), (15, 5)),
        ((1, 6), 0, 5, (3, 2), (10, 5)),
        ((1, 6), 0, 5, (6,), (5, 0)),
        ((6, 1), 7, 0, (2, 3), (21, 7)),
        ((6, 1), 7, 0, (6,), (7, 0)),
        ((2, 3), 12, 4, (6,), (4, 0)),
        ((2, 3), 12, 4, (3, 2), (8, 4)),
        ((2, 3), 12, 4, (1, 6), (24, 4)),
    ],
)
def test_linearly_iterable_sources_reshape_as_views(shape, rs, cs, new, want):
    src = Tensor("x", shape, row_stride=rs if rs else -1, col_stride=cs if cs else -1)
    assert src.can_reshape_as_view(new)
    v = src.reshape_view(new, name="v")
    assert v.buffer_key == "x" and v.shape == new and (v.row_stride, v.col_stride) == want


def test_linear_step():
    assert Tensor("x", (4, 8)).linear_step() == 1
    assert Tensor("x", (4, 8)).transpose("xt").linear_step() is None
    assert Tensor("x", (1, 6), col_stride=5, row_stride=1).linear_step() == 5
    assert Tensor("x", (6, 1), row_stride=7, col_stride=1).linear_step() == 7
    assert Tensor("x", (2, 3), row_stride=12, col_stride=4).linear_step() == 4
    assert Tensor("x", (2, 3), row_stride=10, col_stride=1).linear_step() is None


def test_view_chains_stay_views():
    ops = Operations()
    ops.input("X", shape=(64, 1))
    ops.transpose("X", out="Xt")
    assert ops.reshape("Xt", (64,), out="Y").buffer_key == "X" and ops.build() == []
    ops = Operations()
    ops.input("A", shape=(8, 16))
    ops.transpose("A", out="At")
    att = ops.transpose("At", out="Att")
    assert ops.build() == [] and att.shape == (8, 16) and (att.row_stride, att.col_stride) == (16, 1)
    ops = Operations()
    ops.input("X", shape=(8, 16))
    ops.reshape("X", (128,), out="Xf")
    ops.reshape("Xf", (4, 32), out="Xr")
    assert ops.build() == [] and ops.tensors["Xr"].buffer_key == "X"


@pytest.mark.parametrize("new", [(128,), (4, 32), (32, 4)])
def test_reshape_of_transpose_copies(new):
    ops = Operations()
    ops.input("X", shape=(8, 16))
    ops.transpose("X", out="Xt")
    out = ops.reshape("Xt", new, out="Y")
    (op,) = ops.build()
    assert isinstance(op, ShapeOp) and op.input.name == "Xt" and op.out.name == "Y" and out.buffer_key == "Y"


def test_reshape_errors_and_followups():
    ops = Operations()
    ops.input("X", shape=(8, 16))
    with pytest.raises(ValueError, match="element-count"):
        ops.reshape("X", (9, 16), out="bad")
    ops.transpose("X", out="Xt")
    with pytest.raises(ValueError, match="rank"):
        ops.reshape("Xt", (2, 4, 16), out="bad")
    assert ops.reshape("Xt", (16, 8), out="same").buffer_key == "X"
    ops.reshape("Xt", (128,), out="Y")
    ops.reshape("Y", (16, 8), out="Yr")
    assert sum(isinstance(o, ShapeOp) for o in ops.build()) == 1 and ops.tensors["Yr"].buffer_key == "Y"
    ops = Operations()
    ops.input("A", shape=(8, 16))
    ops.input("At", shape=(16, 8))
    with pytest.raises(ValueError, match="already declared"):
        ops.transpose("A", out="At")


def test_shape_op_kernels():
    ops = Operations()
    ops.input("X", shape=(8, 16))
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", (128,), out="Y")
    (v,) = fuse(ops.build())
    assert assemble(v).strategy is FusionStrategy.STANDALONE_SHAPE and len(v.ops) == 1
    ops = Operations()
    ops.input("A", shape=(8, 16))
    ops.input("B", shape=(16, 8))
    ops.matmul(a="A", b="B", out="C")
    ops.transpose("C", out="Ct")
    ops.reshape("Ct", (64,), out="Cf")
    vs = fuse(ops.build())
    assert {assemble(v).strategy for v in vs} == {FusionStrategy.STANDALONE_MATMUL, FusionStrategy.STANDALONE_SHAPE}


def test_shape_kernel_strides_and_launch():
    ops = Operations()
    ops.input("X", shape=(4, 8))
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", (32,), out="Y")
    g = assemble(fuse(ops.build())[0])
    src = g.kernel.source
    # a transposed view (row stride 1, column stride 8): LDS-tiled transpose
    # reading the owner's buffer along its contiguous axis, 128-bit wide,
    # streaming loads and device-scope stores; 128 x 64 tiles, odd LDS pitch
    assert "mt_ld4_nt(g_X + (size_t)(j0 + jj) * 8u + i0 + li)" in src
    assert "mt_st4_wt(g_Y + (size_t)(i0 + ii) * 4u + j0 + sj" in src
    assert "__shared__ alignas(16) float copy_tile[64][129];" in src
    assert g.bindings == ("X", "Y") and g.dims == (32,)
    assert hip_backend.compile_only(src) > 0
    ops = Operations()  # 13 x 10 transposed view: scalar tiles
    ops.input("X", shape=(10, 13))
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", (130,), out="Y")
    src = assemble(fuse(ops.build())[0]).kernel.source
    assert "g_X[(size_t)j * 13u + i]" in src and "mt_ld4" not in src.split('extern "C"')[1]
    assert hip_backend.compile_only(src) > 0
    # any other strides: one lane per element through the strides
    from compute.copy.copy import StridedCopyFragment
    from compute.fragments import CodegenContext

    frag = StridedCopyFragment("g_X", "g_Y", 12, 4, 3, input_rows=2)
    text = frag.render(CodegenContext(function_name="k", buffers=(), dims=("N",), tg_x=256, tg_y=1))
    assert "(size_t)in_row * 12u + (size_t)in_col * 4u" in text
    assert "global_idx / 3u" in text and "global_idx % 3u" in text and "const unsigned global_idx" in text
    ops = Operations()
    ops.input("X", shape=(10, 13))
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", (130,), out="Y")
    g = assemble(fuse(ops.build())[0])
    assert g.grid == (1, 1, 1) and g.threads == (512, 1, 1) and g.dims == (130,)  # transpose tiles on 512 lanes


def test_transposed_matmul_operand_reads_the_owner_buffer():
    """A^T @ B binds A's buffer and loads it along its contiguous axis
    (reference: the load uses strides (1, 64); gfx950: a row-vector loader
    with column stride 64)."""
    ops = Operations()
    ops.input("A", shape=(32, 64))
    ops.input("B", shape=(32, 16))
    ops.transpose("A", out="At")
    ops.matmul(a="At", b="B", out="C")
    (v,) = fuse(ops.build())
    g = assemble(v)
    src = g.kernel.source
    assert g.bindings[0] == "A"
    assert "const float* __restrict__ g_A" in src and "g_At" not in src
    assert "mt_tile_rowvec<32, 32, 64> ld_A_tile;" in src
    assert "ld_A_tile.template fetch<true>(g_A, 64, tile_m0, k_chunk" in src


def test_reshape_view_feeds_matmul_metadata():
    ops = Operations()
    ops.input("X", shape=(4, 8))
    v = ops.reshape("X", (2, 16), out="Xr")
    assert ops.build() == [] and v.buffer_key == "X" and (v.row_stride, v.col_stride) == (16, 1)
