"""The multi-anchor merge-chain extension (``fusion.MULTI_ANCHOR_MERGE_CHAINS``,
off by default): two matmuls merged through a chain of elementwise ops --
the MLP gate silu(X @ W1) * (X @ W2) -- become one multi-anchor kernel.
With the flag off every partition is the reference's."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.orchestrator import Operations, fusion
from metellus_amd.orchestrator.kernel_group import FusionStrategy
from metellus_amd.runtime import hip_backend
from tests import gpu_cases


def _groups(ops, flag, monkeypatch):
    monkeypatch.setattr(fusion, "MULTI_ANCHOR_MERGE_CHAINS", flag)
    return compile_program(ops)


def _mlp_variant(tail=None, extra_out=None):
    """C4's gate at a small size; ``tail`` edits the program after h1, h2."""
    rng = np.random.default_rng(0)
    ops = Operations()
    for name, shape in (("X", (64, 32)), ("W1", (32, 96)), ("W2", (32, 96)), ("W3", (96, 32)), ("b", (64, 96))):
        ops.from_numpy(rng.standard_normal(shape).astype(np.float32), name)
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="X", b="W2", out="h2")
    (tail or _silu_gate)(ops)
    ops.matmul(a="z", b="W3", out="out")
    if extra_out:
        ops.elementwise("mul", out="o2", operands=(extra_out, 2.0))
    return ops


def _silu_gate(ops):
    _silu_gate_to("z", ops)


def test_reference_partition_with_the_flag_off(monkeypatch):
    gs = _groups(gpu_cases.mlp_block(256, 128, 512), False, monkeypatch)
    assert [g.strategy for g in gs] == [
        FusionStrategy.STANDALONE_MATMUL,
        FusionStrategy.STANDALONE_MATMUL,
        FusionStrategy.ELEMENTWISE_CHAIN,
        FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
    ]


def test_mlp_gate_becomes_one_diamond(monkeypatch):
    gs = _groups(gpu_cases.mlp_block(256, 128, 512), True, monkeypatch)
    assert [g.strategy for g in gs] == [FusionStrategy.DIAMOND_SHARED, FusionStrategy.STANDALONE_MATMUL]
    d, m = gs
    assert [op.out.name for op in d.ops] == ["h1", "h2", "n", "e", "p", "s", "g", "z"]
    assert d.bindings == ("X", "W1", "W2", "z") and m.bindings == ("z", "W3", "out")
    src = d.kernel.source
    body = src[src.index("float merge(float s0, float s1)"):]
    body = body[: body.index("}")]
    # the chain in program order over the two accumulators: s0 = h1, s1 = h2
    for line in ("const float v0 = -(s0);", "const float v1 = expf((v0));", "const float v2 = (v1) + (1.0f);",
                 "const float v3 = 1.0f / (v2);", "const float v4 = (s0) * (v3);", "const float v5 = (v4) * (s1);",
                 "return v5;"):
        assert line in body, line
    assert all(hip_backend.compile_only(g.kernel.source) > 0 for g in gs)


def test_distinct_a_operands_take_two_mainloops(monkeypatch):
    rng = np.random.default_rng(1)
    ops = Operations()
    for name, shape in (("X", (64, 32)), ("Y", (64, 48)), ("W1", (32, 96)), ("W2", (48, 96))):
        ops.from_numpy(rng.standard_normal(shape).astype(np.float32), name)
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="Y", b="W2", out="h2")
    ops.elementwise("max", out="r", operands=("h1", 0.0))
    ops.elementwise("mul", out="z", operands=("r", "h2"))
    (g,) = _groups(ops, True, monkeypatch)
    assert g.strategy is FusionStrategy.MULTI_PRODUCER_CONVERGENT
    assert g.bindings == ("X", "W1", "Y", "W2", "z") and hip_backend.compile_only(g.kernel.source) > 0


def test_one_op_merge_stays_with_the_reference_pass(monkeypatch):
    on = _groups(gpu_cases.mlp_block(256, 128, 512, diamond=True), True, monkeypatch)
    off = _groups(gpu_cases.mlp_block(256, 128, 512, diamond=True), False, monkeypatch)
    assert [g.strategy for g in on] == [g.strategy for g in off] == [FusionStrategy.DIAMOND_SHARED]
    assert on[0].kernel.source == off[0].kernel.source


def _gate_with_bias(ops):
    _silu_gate_to("g2", ops)
    ops.elementwise("add", out="z", operands=("g2", "b"))


def _silu_gate_to(out, ops):
    ops.elementwise("negate", out="n", operands=("h1",))
    ops.elementwise("exp", out="e", operands=("n",))
    ops.elementwise("add", out="p", operands=("e", 1.0))
    ops.elementwise("recip", out="s", operands=("p",))
    ops.elementwise("mul", out="g", operands=("h1", "s"))
    ops.elementwise("mul", out=out, operands=("g", "h2"))


@pytest.mark.parametrize(
    "case",
    [
        "external tensor in the chain",  # z = gate + b: the merge would read b
        "intermediate read outside",  # s is also read after the matmul
    ],
)
def test_chains_that_do_not_fuse(case, monkeypatch):
    if case == "external tensor in the chain":
        ops = _mlp_variant(_gate_with_bias)
    else:
        ops = _mlp_variant(extra_out="s")
    on = _groups(ops, True, monkeypatch)
    assert all(g.strategy is not FusionStrategy.DIAMOND_SHARED for g in on)
    off = _groups(ops, False, monkeypatch)
    assert [g.strategy for g in on] == [g.strategy for g in off]


def test_merge_before_the_second_matmul_does_not_fuse(monkeypatch):
    rng = np.random.default_rng(2)
    ops = Operations()
    for name, shape in (("X", (64, 32)), ("W1", (32, 96)), ("W2", (32, 96))):
        ops.from_numpy(rng.standard_normal(shape).astype(np.float32), name)
    ops.matmul(a="X", b="W1", out="h1")
    ops.elementwise("negate", out="n", operands=("h1",))  # before h2 in program order
    ops.matmul(a="X", b="W2", out="h2")
    ops.elementwise("mul", out="z", operands=("n", "h2"))
    on = _groups(ops, True, monkeypatch)
    off = _groups(ops, False, monkeypatch)
    assert [g.strategy for g in on] == [g.strategy for g in off]
