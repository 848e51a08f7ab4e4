"""The known-answer fixtures (tests/golden/kats.npz) through the full
pipeline on the GPU: each case is a one-op program run by ``api.run``."""

import numpy as np
import pytest

from metellus_amd.api import run
from metellus_amd.orchestrator import Operations
from tests.test_oracle import KATS, kat_ok

pytestmark = pytest.mark.gpu


def _program(case):
    op = str(case["op"])
    ops = Operations()
    ops.from_numpy(np.ascontiguousarray(case["x"], dtype=np.float32), "x")
    if op.startswith("reduce_"):
        ops.reduction(op[len("reduce_"):], out="out", x="x")
        return ops
    operands = ["x"]
    if "y" in case:
        ops.from_numpy(np.ascontiguousarray(case["y"], dtype=np.float32), "y")
        operands.append("y")
    if "scalar" in case:
        operands.append(float(case["scalar"]))
    if "cond" in case:
        ops.from_numpy(np.ascontiguousarray(case["cond"], dtype=np.float32), "cond")
        operands.append("cond")
    ops.elementwise(op, out="out", operands=tuple(operands))
    return ops


@pytest.mark.parametrize("name", sorted(KATS))
def test_gpu_known_answers(name):
    case = KATS[name]
    res = run(_program(case))
    assert kat_ok(case, res.env["out"]), (name, res.env["out"], case["expected"])
