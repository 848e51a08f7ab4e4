"""The reference's correctness sweep (sandbox.py, 188 registered probes)
and its 10 end-to-end scenarios (runner.py), restated in ``tests/probes.py``.  Without a GPU: every probe fuses,
assembles, schedules and compiles for gfx950, and each output the probe
checks is materialised and downloaded by the schedule (fused intermediates
are not).  Results are checked on the GPU (``test_gpu_probes.py``)."""

import pytest

from metellus_amd.api import compile_program
from metellus_amd.orchestrator.scheduler import schedule
from metellus_amd.runtime import hip_backend
from metellus_amd.runtime.program import Download
from tests.probes import PROBES, SCENARIOS, build, build_scenario


def test_all_registered_reference_probes_are_restated():
    assert len(PROBES) == 188
    assert len(SCENARIOS) == 10


def _compiles_and_downloads(p):
    groups = compile_program(p.ops)
    downloads = {f.into for f in schedule(p.ops, groups).fragments if isinstance(f, Download)}
    assert set(p.checks) <= downloads, sorted(set(p.checks) - downloads)
    for g in groups:
        assert hip_backend.compile_only(g.kernel.source) > 0


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_scenario_compiles_and_downloads_its_checks(name):
    _compiles_and_downloads(build_scenario(name))


@pytest.mark.parametrize("name", sorted(PROBES))
def test_probe_compiles_and_downloads_its_checks(name):
    _compiles_and_downloads(build(name))
