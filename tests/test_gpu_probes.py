"""The reference's correctness sweep (sandbox.py, 188 probes) on the
MI355X: each probe's program runs through ``api.run`` and every output it
checks is compared with the CPU oracle on the same inputs.  Bar: the
reference's own, rtol = atol = 1e-3 with NaN equal to NaN
(sandbox.py:40-49); outputs the probe marks exact (IEEE-exact elementwise
chains, comparisons, max/min reductions, integer-valued sums, NaN/inf
cases) must match bit for bit (NaN matching NaN).  The 10 runner.py
scenarios use that file's bar, rtol = 1e-3, atol = 1e-2 (runner.py:87-102)."""

import numpy as np
import pytest

from metellus_amd.api import run
from oracle.ir_eval import evaluate
from tests.probes import PROBES, SCENARIOS, build, build_scenario

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", sorted(PROBES))
def test_probe(name):
    p = build(name)
    env = run(p.ops).env
    ref = evaluate(p.ops)
    for t in p.checks:
        got, want = np.asarray(env[t]), np.asarray(ref[t], dtype=np.float32)
        assert got.shape == want.shape, (t, got.shape, want.shape)
        if t in p.exact:
            np.testing.assert_array_equal(got, want, err_msg=t)
        else:
            np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-3, equal_nan=True, err_msg=t)


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_scenario(name):
    p = build_scenario(name)
    env = run(p.ops).env
    ref = evaluate(p.ops)
    for t in p.checks:
        got, want = np.asarray(env[t]), np.asarray(ref[t], dtype=np.float32)
        assert got.shape == want.shape, (t, got.shape, want.shape)
        if t in p.exact:
            np.testing.assert_array_equal(got, want, err_msg=t)
        else:
            np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-2, err_msg=t)
