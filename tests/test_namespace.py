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


def test_run_kernel_checks_its_slots_before_compiling():
    """run_kernel's slots are a Buffer, an int handle or a writeable
    C-contiguous ndarray (its contents are written back in place); anything
    else is refused before the kernel is compiled or a buffer allocated, so
    these checks run without a GPU."""
    import numpy as np
    import pytest

    import metal_backend

    src, fn = "not compiled", "k"
    with pytest.raises(TypeError, match="a slot is a Buffer, an int handle or an ndarray"):
        metal_backend.run_kernel(src, fn, ["buf"], (1, 1, 1), (64, 1, 1))
    with pytest.raises(TypeError, match="got list"):
        metal_backend.run_kernel(src, fn, [[1.0, 2.0]], (1, 1, 1), (64, 1, 1))
    strided = np.zeros((4, 4), np.float32)[:, ::2]
    with pytest.raises(ValueError, match="C-contiguous and writeable"):
        metal_backend.run_kernel(src, fn, [strided], (1, 1, 1), (64, 1, 1))
    frozen = np.zeros(8, np.float32)
    frozen.flags.writeable = False
    with pytest.raises(ValueError, match="C-contiguous and writeable"):
        metal_backend.run_kernel(src, fn, [frozen], (1, 1, 1), (64, 1, 1))
