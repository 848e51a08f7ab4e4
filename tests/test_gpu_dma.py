"""Direct-to-LDS operand loads (``mt_tile_dma``) against the register path
on the GPU: the two only move data differently (the MFMAs see the same
values in the same order), so every output must be bit-identical -- plain,
persistent with a stream-K last round, K^T stored n-major, the diamond's
two B chunks, a gather prologue on A beside a directly loaded B, and
batched heads -- and within the matmul bar of float64."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import compile_program, run, run_batch
from metellus_amd.compute.matmul import config
from metellus_amd.orchestrator.assembly import matmul as mm
from oracle.ir_eval import evaluate, matmul_tolerance
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def _both(make, monkeypatch, outputs):
    """(register-path env, direct-to-LDS env, direct-to-LDS groups), on the
    LDS-tiled kernels (the K-resident kernel loads B directly either way)."""
    monkeypatch.setattr(mm, "K_RESIDENT", False)
    monkeypatch.setattr(mm, "DMA_LOADS", False)
    ref = run(make(), outputs=outputs).env
    monkeypatch.setattr(mm, "DMA_LOADS", True)
    ops = make()
    res = run(ops, outputs=outputs)
    return ref, res.env, res.groups, ops


@pytest.mark.parametrize("mkn", [(512, 512, 512), (256, 1024, 768), (4096, 256, 4096)])
def test_plain_matmul_bit_identical(mkn, monkeypatch):
    make = lambda: gpu_cases.plain_matmul(*mkn, seed=21)
    ref, env, groups, ops = _both(make, monkeypatch, ("C",))
    assert "mt_tile_dma<" in groups[0].kernel.source
    np.testing.assert_array_equal(env["C"], ref["C"])
    err = np.abs(env["C"].astype(np.float64) - evaluate(ops)["C"])
    assert np.all(err <= matmul_tolerance(ops.uploads["A"], ops.uploads["B"]) + 1e-30)


def test_stream_k_bit_identical(monkeypatch):
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 7)  # 15 tiles on 7 workgroups: stream-K last round
    make = lambda: gpu_cases.plain_matmul(768, 512, 1280, seed=22)
    ref, env, groups, ops = _both(make, monkeypatch, ("C",))
    g = groups[0]
    assert g.grid == (7, 1, 1) and g.kernel.workspace_bytes > 0 and "mt_tile_dma<" in g.kernel.source
    np.testing.assert_array_equal(env["C"], ref["C"])
    from metellus_amd.runtime import hip_backend

    hip_backend.check_workspace()


def test_transposed_b_and_prologue_a(monkeypatch):
    """Attention head: S = Q @ K^T (K^T n-major) and O = (e / s1) @ V (gather
    prologue on A through registers, V loaded directly)."""
    make = lambda: gpu_cases.attention_head(512, 64, seed=23)
    ref, env, groups, ops = _both(make, monkeypatch, ("Ss", "e", "s1", "O"))
    src = {g.kernel.function_name: g.kernel.source for g in groups}
    assert "true, true>(" in src["matmul_S_fused"] and "mt_tile_dma<" in src["matmul_O_fused"]
    for name in ("Ss", "e", "s1", "O"):
        np.testing.assert_array_equal(env[name], ref[name], err_msg=name)


def test_diamond_and_literal_mlp(monkeypatch):
    make = lambda: gpu_cases.mlp_block(512, 256, 512, seed=24, diamond=True)
    ref, env, groups, _ = _both(make, monkeypatch, ("z",))
    assert groups[0].kernel.source.count("mt_tile_dma<") == 3  # A and both B chunks
    np.testing.assert_array_equal(env["z"], ref["z"])
    # same k-chunk width on both paths (the register path narrows the chunks
    # of a full-size gather prologue to 16 by default), so the sums match
    monkeypatch.setattr(mm, "GATHER_TILE_K", 32)
    make = lambda: gpu_cases.mlp_block(256, 256, 512, seed=25)
    ref, env, groups, _ = _both(make, monkeypatch, ("h1", "h2", "out"))
    for name in ("h1", "h2", "out"):
        np.testing.assert_array_equal(env[name], ref[name], err_msg=name)


def test_batched_heads(monkeypatch):
    heads = 4
    progs = lambda: [gpu_cases.attention_head(256, 64, seed=26, head=h, heads=heads) for h in range(heads)]
    monkeypatch.setattr(mm, "DMA_LOADS", False)
    ref = run_batch(progs(), outputs=("Ss", "O"))
    monkeypatch.setattr(mm, "DMA_LOADS", True)
    p = progs()
    assert "mt_tile_dma<" in compile_program(p[0], batch=heads)[0].kernel.batched().source
    res = run_batch(p, outputs=("Ss", "O"))
    for a, b in zip(ref, res):
        np.testing.assert_array_equal(b.env["Ss"], a.env["Ss"])
        np.testing.assert_array_equal(b.env["O"], a.env["O"])
