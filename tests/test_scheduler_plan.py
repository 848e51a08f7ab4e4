"""Runtime plans built by ``schedule`` (no kernels run): upload / allocate /
dispatch / download / free order and the validation errors (the
host-side assertions of the reference's tests/test_scheduler.py)."""

import numpy as np
import pytest

from orchestrator import Operations
from orchestrator.aliasing import alias_group
from orchestrator.assembly import assemble
from orchestrator.fusion import fuse
from orchestrator.scheduler import schedule
from metellus_amd.api import compile_program
from runtime import Allocate, Dispatch, Download, Free, FromNumpy, Kernel


def _groups(ops):
    return tuple(alias_group(assemble(v)) for v in fuse(ops.build()))


def _kinds(rt):
    return [type(s).__name__ for s in rt.fragments]


def _mm(ops, shape=(32, 16), shape_b=(16, 24)):
    rng = np.random.default_rng(0)
    ops.from_numpy(rng.standard_normal(shape).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal(shape_b).astype(np.float32), "B")


def test_fused_intermediate_never_allocated():
    ops = Operations()
    _mm(ops)
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="D", operands=("C", 0.0))
    rt = schedule(ops, _groups(ops))
    allocs = [s.name for s in rt.fragments if isinstance(s, Allocate)]
    downloads = [s.into for s in rt.fragments if isinstance(s, Download)]
    assert allocs == ["D"] and downloads == ["D"]
    assert _kinds(rt)[:2] == ["FromNumpy", "FromNumpy"]


def test_last_use_download_and_free():
    ops = Operations()
    _mm(ops)
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="D", operands=("C", 0.0))
    ops.elementwise("absolute", out="E", operands=("C",))
    groups = _groups(ops)
    assert len(groups) == 3
    rt = schedule(ops, groups)
    steps = rt.fragments
    dispatch_at = [i for i, s in enumerate(steps) if isinstance(s, Dispatch)]
    c_download = next(i for i, s in enumerate(steps) if isinstance(s, Download) and s.into == "C")
    assert c_download > dispatch_at[2]  # C dies after its last reader (E's kernel)
    frees = [s.name for s in steps if isinstance(s, Free)]
    assert set(frees) == {"A", "B"}
    a_free = next(i for i, s in enumerate(steps) if isinstance(s, Free) and s.name == "A")
    assert a_free > dispatch_at[0] and a_free < dispatch_at[1]


def test_views_download_before_owner_with_strides():
    ops = Operations()
    rng = np.random.default_rng(4)
    ops.from_numpy(rng.standard_normal((8, 6)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((8, 5)).astype(np.float32), "B")
    ops.transpose("A", out="At")
    ops.matmul(a="At", b="B", out="C")
    rt = schedule(ops, _groups(ops))
    views = [s for s in rt.fragments if isinstance(s, Download) and s.into == "At"]
    assert len(views) == 1 and (views[0].row_stride, views[0].col_stride) == (1, 6)


def test_profile_time_keys():
    ops = Operations()
    _mm(ops)
    ops.matmul(a="A", b="B", out="C")
    rt = schedule(ops, _groups(ops), profile=True)
    assert [s.time_key for s in rt.fragments if isinstance(s, Dispatch)] == ["t_0"]


def test_kernels_primed_before_dispatch():
    ops = Operations()
    _mm(ops)
    ops.matmul(a="A", b="B", out="C")
    rt = schedule(ops, _groups(ops))
    k = next(i for i, s in enumerate(rt.fragments) if isinstance(s, Kernel))
    d = next(i for i, s in enumerate(rt.fragments) if isinstance(s, Dispatch))
    assert k < d


def test_missing_and_extra_uploads():
    ops = Operations()
    ops.input("A", shape=(8, 8))
    ops.input("B", shape=(8, 8))
    ops.matmul(a="A", b="B", out="C")
    with pytest.raises(ValueError, match="no from_numpy upload"):
        schedule(ops, _groups(ops))
    ops = Operations()
    _mm(ops)
    ops.from_numpy(np.zeros((2, 2), dtype=np.float32), "unused")
    ops.matmul(a="A", b="B", out="C")
    with pytest.raises(ValueError, match="do not correspond"):
        schedule(ops, _groups(ops))


def test_view_of_produced_buffer_needs_no_upload():
    ops = Operations()
    ops.from_numpy(np.ones((4, 8), dtype=np.float32), "X")
    ops.reduction("sum", out="s", x="X")
    ops.reshape("s", (4, 1), out="sv")
    ops.elementwise("div", out="p", operands=("X", "sv"), y_broadcast="col")
    rt = schedule(ops, _groups(ops))
    assert [s.name for s in rt.fragments if isinstance(s, FromNumpy)] == ["X"]


def test_outputs_limits_downloads_and_frees_the_rest():
    from tests.gpu_cases import softmax

    ops = softmax(32, 100)
    groups = compile_program(ops)
    full = schedule(ops, groups).fragments
    only = schedule(ops, groups, outputs=["p"]).fragments
    downloaded = lambda steps: sorted(f.into for f in steps if isinstance(f, Download))  # noqa: E731
    freed = lambda steps: sorted(f.name for f in steps if isinstance(f, Free))  # noqa: E731
    assert "p" in downloaded(full) and len(downloaded(full)) > 1
    assert downloaded(only) == ["p"]
    # every other produced buffer is freed at its last use instead
    assert set(freed(only)) >= {g.bindings[-1] for g in groups if g.bindings[-1] != "p"} - set(ops.uploads)


def test_outputs_must_be_materialised():
    import pytest

    from tests.gpu_cases import sigmoid_chain

    ops = sigmoid_chain(16, 16)
    groups = compile_program(ops)
    with pytest.raises(ValueError, match="not materialised"):
        schedule(ops, groups, outputs=["t1"])  # fused into the chain kernel
    with pytest.raises(ValueError, match="unknown output"):
        schedule(ops, groups, outputs=["nope"])
