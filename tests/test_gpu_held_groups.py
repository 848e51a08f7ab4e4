"""The held-group mainloop on the GPU: carrying each chunk's last group of 4
k-steps over the barrier adds every product in the same k order, so every
output is bit-identical to the plain mainloop's -- aligned, ragged (a
partial last chunk, bounds checks), persistent with stream-K, a prologue
division taking either of its two k loops, and batched attention."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run, run_batch
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly import matmul as mm
from tests import gpu_cases

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _lds_tiled(monkeypatch):
    """Matmuls 128 columns wide on the LDS-tiled mainloop these tests are
    about (they take the row-owning-wave kernel by default)."""
    monkeypatch.setattr(mm, "ROW_WAVES", False)


def _divided(M: int, K: int, N: int, plain: bool) -> Operations:
    """Y = (E / s[row]) @ V; with ``plain`` False some rows' divisors (below
    1, zero, subnormal) send their tiles down the per-element k loop."""
    rng = np.random.default_rng(43)
    e = rng.random((M, K), dtype=np.float32) + 0.1
    s = (rng.random(M, dtype=np.float32) * 100.0 + 1.0).astype(np.float32)
    if not plain:
        s[[5, 260, 261]] = np.array([0.5, 0.0, 1e-40], dtype=np.float32)
    ops = Operations()
    ops.from_numpy(e, "E")
    ops.from_numpy(s, "s")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "V")
    ops.reshape("s", (M, 1), out="sv")
    ops.elementwise("div", out="P", operands=("E", "sv"), y_broadcast="col")
    ops.matmul(a="P", b="V", out="Y")
    return ops


_CASES = {
    "aligned 1024^3": lambda: gpu_cases.plain_matmul(1024, 1024, 1024),
    "ragged 300x777x1000": lambda: gpu_cases.plain_matmul(300, 777, 1000),
    "persistent stream-K 4096x4096x11008": lambda: gpu_cases.plain_matmul(4096, 4096, 11008),
    "prologue division, plain loop": lambda: _divided(512, 1024, 128, True),
    "prologue division, per-element loop": lambda: _divided(512, 1024, 128, False),
}


@pytest.mark.parametrize("case", list(_CASES))
def test_held_matches_plain_mainloop(case, monkeypatch):
    out = "Y" if "division" in case else "C"
    got = {}
    for held in (True, False):
        monkeypatch.setattr(mm, "HELD_GROUPS", held)
        print(f"held groups: {case} held={held}", flush=True)
        res = run(_CASES[case](), outputs=(out,))
        body = res.groups[-1].kernel.source.split('extern "C"')[-1]
        assert ("mt_mfma_tile_held<" in body) == held, case
        if "stream-K" in case:
            assert "mt_sk_wait(" in body
        got[held] = res.env[out]
    np.testing.assert_array_equal(got[True], got[False], err_msg=case)
    if "per-element" not in case:
        assert np.all(np.isfinite(got[True]))


def test_batched_attention_heads(monkeypatch):
    """C5 at 2048 x 128 for 4 heads: the P @ V kernel holds a group in both
    of its k loops; every output matches the plain mainloop's."""
    heads = 4
    outs = ("Ss", "m1", "e", "s1", "O")
    make = lambda: [gpu_cases.attention_head(2048, 128, head=h, heads=heads) for h in range(heads)]
    got = {}
    for held in (True, False):
        monkeypatch.setattr(mm, "HELD_GROUPS", held)
        print(f"held groups: attention heads held={held}", flush=True)
        res = run_batch(make(), outputs=outs)
        assert ("mt_mfma_tile_held<" in res[0].groups[-1].kernel.source.split('extern "C"')[-1]) == held
        got[held] = res
    for h in range(heads):
        for name in outs:
            np.testing.assert_array_equal(got[True][h].env[name], got[False][h].env[name], err_msg=f"head {h} {name}")
