"""``run_batch``: structurally identical programs (attention heads) run with
one batched launch per fused kernel; results per program must match the
oracle exactly as single runs do."""

import numpy as np
import pytest

from metellus_amd.api import BatchRunner, run, run_batch
from oracle.ir_eval import evaluate
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def test_attention_heads_batched():
    heads = 4
    progs = [gpu_cases.attention_head(256, 64, head=h, heads=heads) for h in range(heads)]
    runner = BatchRunner(progs)
    assert runner.batched
    results = runner.run()
    for ops, res in zip(progs, results):
        ref = evaluate(ops)
        np.testing.assert_allclose(res.env["O"], ref["O"], rtol=1e-3, atol=1e-4)
        np.testing.assert_allclose(res.env["e"], ref["e"], rtol=1e-4, atol=1e-6)
        assert "P" not in res.env  # fused into the P@V prologue


def test_batched_softmax_matches_single_runs_bitwise():
    progs = [gpu_cases.softmax(48, 300, seed=s) for s in range(3)]
    batched = run_batch(progs)
    for ops, res in zip(progs, batched):
        single = run(ops)
        for name in ("m1", "e", "s1", "p"):
            np.testing.assert_array_equal(res.env[name], single.env[name])


def test_mismatched_programs_fall_back_to_sequential():
    progs = [gpu_cases.sigmoid_chain(16, 32), gpu_cases.sigmoid_chain(24, 40)]
    runner = BatchRunner(progs)
    assert not runner.batched
    for ops, res in zip(progs, runner.run()):
        np.testing.assert_allclose(res.env["out"], evaluate(ops)["out"], rtol=1e-5, atol=1e-5)
