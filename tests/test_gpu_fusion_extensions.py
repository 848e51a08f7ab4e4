"""The multi-anchor merge-chain extension on the GPU: the MLP block with its
gate silu(X @ W1) * (X @ W2) in one multi-anchor kernel gives the same bits
as the reference's 4-kernel partition (same k-chunk order in every matmul,
the same IEEE ops in the same order in the gate)."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run
from metellus_amd.orchestrator import fusion
from metellus_amd.orchestrator.assembly import matmul as mm
from tests import gpu_cases

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mdh", [(256, 256, 512), (512, 128, 768)])
def test_mlp_gate_extension_matches_the_reference_partition(mdh, monkeypatch):
    # the literal (h1*s*h2) @ W3 loads A through registers with 16-wide chunks
    # by default; 32-wide ones pair the k terms like the plain matmul
    monkeypatch.setattr(mm, "GATHER_TILE_K", 32)
    make = lambda: gpu_cases.mlp_block(*mdh, seed=31)
    monkeypatch.setattr(fusion, "MULTI_ANCHOR_MERGE_CHAINS", False)
    lit = run(make(), outputs=("h1", "s", "h2", "out"))
    monkeypatch.setattr(fusion, "MULTI_ANCHOR_MERGE_CHAINS", True)
    ext = run(make(), outputs=("z", "out"))
    assert len(lit.groups) == 4 and len(ext.groups) == 2
    h1, s, h2 = lit.env["h1"], lit.env["s"], lit.env["h2"]
    z = (h1 * s) * h2  # the literal W3 kernel's A operand: two IEEE multiplies
    np.testing.assert_array_equal(ext.env["z"], z)
    np.testing.assert_array_equal(ext.env["out"], lit.env["out"])
