"""Test configuration.

* ``gpu`` marks tests that launch kernels on an MI355X (run with -m gpu);
  everything else runs on a CPU-only machine.
* The reference's top-level module names (``orchestrator``, ``compute``,
  ``runtime``, ...) are installed as aliases of ``metellus_amd`` so the
  restated reference tests import exactly as the reference's do.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import metellus_amd  # noqa: E402

metellus_amd.install_reference_namespace()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs kernels through the HIP shim)")
