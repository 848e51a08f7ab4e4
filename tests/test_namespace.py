"""The reference's module names resolve to this package's modules (same
objects, so isinstance checks and monkeypatches agree)."""

import importlib


def test_aliases_are_the_same_modules():
    for ref, real in [
        ("orchestrator", "metellus_amd.orchestrator"),
        ("orchestrator.fusion", "metellus_amd.orchestrator.fusion"),
        ("orchestrator.assembly", "metellus_amd.orchestrator.assembly"),
        ("compute.elementwise.elementwise", "metellus_amd.compute.elementwise.elementwise"),
        ("memory.memory", "metellus_amd.memory.memory"),
        ("runtime", "metellus_amd.runtime"),
        ("api", "metellus_amd.api"),
        ("metal_backend", "metellus_amd.runtime.hip_backend"),
    ]:
        assert importlib.import_module(ref) is importlib.import_module(real)


def test_reference_style_imports():
    from api import run  # noqa: F401
    from orchestrator import Operations
    from orchestrator.ir import Tensor
    from metellus_amd.orchestrator.ir import Tensor as T2

    assert Tensor is T2
    assert Operations().input("x", (2, 2)).shape == (2, 2)


def test_real_module_spec_is_kept():
    import orchestrator.fusion as f

    assert f.__spec__.name == "metellus_amd.orchestrator.fusion"
