"""The held-group mainloop (``MatmulMainloopFragment.held``): each k-chunk's
last group of 4 k-steps is carried over the barrier into the next chunk.
Checked on the CPU: which kernels get it, the code it renders, and that the
kernels compile."""

from __future__ import annotations

import pytest

from metellus_amd.api import compile_program
from metellus_amd.compute.matmul.matmul import MatmulMainloopFragment
from metellus_amd.orchestrator.assembly import matmul as mm
from metellus_amd.runtime import hip_backend
from tests.gpu_cases import attention_head, mlp_block, plain_matmul


@pytest.fixture(autouse=True)
def _lds_tiled(monkeypatch):
    """C5 P @ V and Q @ K^T on the LDS-tiled mainloop these tests are about
    (they take the row-owning-wave and the K-resident kernels by default)."""
    monkeypatch.setattr(mm, "ROW_WAVES", False)
    monkeypatch.setattr(mm, "K_RESIDENT", False)


def _body(group) -> str:
    return group.kernel.source.split('extern "C"')[-1]


def _bench_kernels():
    mlp = compile_program(mlp_block(4096, 4096, 11008))
    att = compile_program(attention_head(2048, 128, heads=32), batch=32)
    return {
        "gemm": compile_program(plain_matmul(4096, 4096, 4096))[0],
        "h1": mlp[0],
        "w3": mlp[3],
        "s": att[0],
        "o": att[4],
    }


def test_which_kernels_hold_a_group():
    """Many chunks and no spread loads: the 4096^3 GEMM, C4 X @ W1 and C5
    P @ V (both of its k loops); C5 Q @ K^T has 4 chunks and C4 W3 spreads
    its loads, so they keep the plain mainloop."""
    ks = _bench_kernels()
    held = {k: _body(g).count("mt_mfma_tile_held<") for k, g in ks.items()}
    assert held == {"gemm": 1, "h1": 1, "w3": 0, "s": 0, "o": 2}
    for k, g in ks.items():
        b = _body(g)
        assert b.count("mt_mfma_group_run<") == held[k]  # one flush per k loop
        assert ("mt_mfma_tile<" in b) == (held[k] == 0)


def test_rendered_loop():
    """Zeroed group before the loop, carried when kt is past the loop's
    first chunk, flushed after it -- for the plain k loop (from 0) and the
    persistent one (from the item's first chunk)."""
    o = _body(_bench_kernels()["o"])
    assert "mt_mfma_group<2, 1> mt_held0 = {};" in o
    assert "acc, lane, mt_held0, kt > 0u);" in o
    loop_end = o.index("mt_mfma_group_run<2, 1>(mt_held0, acc);")
    assert o.rindex("__syncthreads();", 0, loop_end) > o.index("mt_mfma_tile_held<")
    sk = compile_program(plain_matmul(4096, 4096, 11008))[0]  # persistent, stream-K
    body = _body(sk)
    assert "for (unsigned kt = mt_kb; kt < mt_ke; ++kt)" in body and "mt_sk_wait(" in body
    assert "mt_held0, kt > mt_kb);" in body
    assert hip_backend.compile_only(sk.kernel.source) > 0


def test_few_chunks_or_flag_off(monkeypatch):
    short = compile_program(plain_matmul(1024, 256, 1024))[0]  # 8 chunks
    assert "mt_mfma_tile_held<" not in _body(short)
    monkeypatch.setattr(mm, "HELD_GROUPS", False)
    gemm = compile_program(plain_matmul(4096, 4096, 4096))[0]
    assert "mt_mfma_tile_held<" not in _body(gemm) and "mt_mfma_tile<" in _body(gemm)


def test_held_and_spread_do_not_combine():
    frag = MatmulMainloopFragment(tile_K=32, fragments=(), K_dim_var="K", spread=2, held=True)
    with pytest.raises(ValueError, match="held group and spread loads"):
        frag._held(2)


@pytest.mark.parametrize("name", ["gemm", "h1", "o"])
def test_held_kernels_compile(name):
    g = _bench_kernels()[name]
    src = g.kernel.batched().source if name == "o" else g.kernel.source
    assert hip_backend.compile_only(src) > 0
