"""The C-ABI shim without a GPU: the library loads, exports every symbol
``include/metellus_hip.h`` declares, compiles every kernel family for gfx950
through hiprtc, reports compile errors, and fails loudly (RuntimeError)
where a device is needed but absent.  Compute calls are GPU tests."""

import os
import re

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.runtime import hip_backend
from tests import gpu_cases

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "metellus_hip.h")).read()
    return sorted(set(re.findall(r"\b(mt_[a-z_]+)\s*\(", text)))


def test_header_and_wrapper_agree():
    assert _declared() == sorted(hip_backend.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = hip_backend.library()
    for name in _declared():
        assert hasattr(lib, name), name


def test_last_error_starts_empty_or_string():
    assert isinstance(hip_backend.library().mt_last_error(), bytes)


@pytest.mark.parametrize(
    "build",
    [
        lambda: gpu_cases.sigmoid_chain(64, 64),
        lambda: gpu_cases.softmax(32, 100),
        lambda: gpu_cases.matmul_bias_relu(100, 70, 130),
        lambda: gpu_cases.mlp_block(64, 64, 96),
        lambda: gpu_cases.mlp_block(64, 64, 96, diamond=True),
        lambda: gpu_cases.attention_head(64, 32),
    ],
)
def test_generated_kernels_compile_for_gfx950(build):
    for g in compile_program(build()):
        assert hip_backend.compile_only(g.kernel.source) > 0


def test_compile_error_is_reported():
    with pytest.raises(RuntimeError, match="hiprtc compile failed"):
        hip_backend.compile_only('extern "C" __global__ void k() { this is not c++ }')


def test_device_calls_fail_loudly_without_gpu():
    if hip_backend.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="no HIP device"):
        hip_backend.create_buffer(16)


def test_buffer_validation_before_device():
    with pytest.raises(RuntimeError, match="nbytes must be > 0"):
        hip_backend.create_buffer(0)
    with pytest.raises(ValueError):
        hip_backend.fill_buffer(1, 300)
    with pytest.raises(ValueError, match="C-contiguous"):
        hip_backend.read_buffer(1, np.zeros((4, 4), dtype=np.float32).T)
