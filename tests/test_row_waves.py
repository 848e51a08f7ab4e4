"""The row-owning-wave matmul (``MatmulRowWavesFragment``, ``mt_rw_*``) on the
CPU: which matmuls take it (``assembly.matmul.row_waves``), what the kernel
renders, and that every form compiles."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly import matmul as mm
from metellus_amd.runtime import hip_backend
from tests.gpu_cases import attention_head


def _body(g) -> str:
    return g.kernel.source.split('extern "C"')[-1]


def _program(M=512, K=1024, N=128, prologue="none", epilogue=False, a_view=False, b_view=False) -> Operations:
    rng = np.random.default_rng(5)
    ops = Operations()
    if a_view:
        ops.from_numpy(rng.standard_normal((K, M)).astype(np.float32), "As")
        ops.transpose("As", out="A")
    else:
        ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    if b_view:  # B as a transposed view (K^T-like): read along its columns
        ops.from_numpy(rng.standard_normal((N, K)).astype(np.float32), "Bs")
        ops.transpose("Bs", out="B")
    else:
        ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    a = "A"
    if prologue == "row divisor":
        ops.from_numpy((rng.random(M) + 1.0).astype(np.float32), "s")
        ops.reshape("s", (M, 1), out="sv")
        ops.elementwise("div", out="P", operands=("A", "sv"), y_broadcast="col")
        a = "P"
    elif prologue == "scalar":
        ops.elementwise("mul", out="P", operands=("A", 0.5))
        a = "P"
    elif prologue == "column scale":
        ops.from_numpy(rng.random(K).astype(np.float32), "w")
        ops.reshape("w", (1, K), out="wv")
        ops.elementwise("mul", out="P", operands=("A", "wv"), y_broadcast="row")
        a = "P"
    ops.matmul(a=a, b="B", out="Y")
    if epilogue:
        ops.elementwise("max", out="Z", operands=("Y", 0.0))
    return ops


def _matmul_group(ops):
    return [g for g in compile_program(ops) if g.kernel is not None and "matmul" in g.kernel.function_name][-1]


def test_attention_output_takes_row_waves():
    gs = compile_program(attention_head(2048, 128, heads=32), batch=32)
    o = gs[4]
    assert o.grid == (1, 8, 1) and o.threads == (1024, 1, 1) and o.bindings == ("e", "V", "O", "s1")
    body = o.kernel.batched().source.split('extern "C"')[-1]
    assert "B_tile[2][64][128]" in body and "A_tile" not in body
    assert body.count("mt_rw_chunk(") == 4  # two chunks a trip, plain and per-element loops
    assert "__syncthreads_and(xp(mt_e) ? 1 : 0)" in body and "mt_pq" in body
    assert hip_backend.compile_only(o.kernel.batched().source) > 0
    assert gs[0].kernel is not None and "mt_rw_chunk(" not in _body(gs[0])  # S: 2048 columns


@pytest.mark.parametrize("prologue", ["none", "row divisor", "scalar"])
@pytest.mark.parametrize("epilogue", [False, True])
def test_forms_compile(prologue, epilogue):
    g = _matmul_group(_program(prologue=prologue, epilogue=epilogue))
    body = _body(g)
    assert "mt_rw_chunk(" in body and g.grid == (1, 2, 1)
    assert ("__syncthreads_and" in body) == (prologue == "row divisor")
    assert ("xt(raw, mt_row, 0u)" in body) == (prologue == "scalar")
    assert hip_backend.compile_only(g.kernel.source) > 0


@pytest.mark.parametrize(
    "case",
    [
        dict(N=256), dict(M=300), dict(K=512), dict(K=1088), dict(a_view=True), dict(b_view=True),
        dict(prologue="column scale"),
    ],
)
def test_shapes_that_keep_the_lds_tiled_kernel(case):
    assert "mt_rw_chunk(" not in _body(_matmul_group(_program(**case)))


def test_flag_off(monkeypatch):
    monkeypatch.setattr(mm, "ROW_WAVES", False)
    assert "mt_rw_chunk(" not in _body(_matmul_group(_program()))
