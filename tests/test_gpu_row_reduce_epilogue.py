"""The matmul -> reduction epilogue extension on the GPU: the matmul kernel
that also reduces its output's rows writes the same matmul output as the
reference partition, and a row reduction of exactly those values -- max and
min bit for bit, sum and product within their summation-order bounds -- also
when the program is launched again (the row-block counters reset), for
ragged, persistent and batched launches."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run, run_batch
from metellus_amd.orchestrator import Operations, fusion
from metellus_amd.orchestrator.assembly import matmul as mm
from metellus_amd.orchestrator.kernel_group import FusionStrategy
from oracle.ir_eval import evaluate
from tests import gpu_cases

pytestmark = pytest.mark.gpu

EPS = np.finfo(np.float32).eps


def _program(op: str, M: int, K: int, N: int, seed: int = 11) -> Operations:
    """Y = A @ B, Yc = Y * s + t (a register epilogue), r = op(Yc) over rows,
    and one more reader of Yc.  For product the scale keeps the row products
    finite (values near 1)."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.matmul(a="A", b="B", out="Y")
    scale, shift = (0.5, 0.0) if op != "product" else (1.0 / (8.0 * K), 1.0)
    ops.elementwise("mul", out="Ys", operands=("Y", scale))
    ops.elementwise("add", out="Yc", operands=("Ys", shift))
    ops.reduction(op, out="r", x="Yc")
    ops.elementwise("mul", out="z", operands=("Yc", 2.0))
    return ops


def _check_rows(op: str, r: np.ndarray, yc: np.ndarray) -> None:
    """``r`` against the row reduction of the kernel's own output ``yc``."""
    if op == "max":
        np.testing.assert_array_equal(r, yc.max(axis=1))
    elif op == "min":
        np.testing.assert_array_equal(r, yc.min(axis=1))
    elif op == "sum":
        ref = yc.astype(np.float64).sum(axis=1)
        bound = 64 * EPS * np.abs(yc).astype(np.float64).sum(axis=1)  # a fixed tree of depth < 64
        assert np.all(np.abs(r - ref) <= bound), np.max(np.abs(r - ref) / bound)
    else:
        ref = np.prod(yc.astype(np.float64), axis=1)
        assert np.all(np.isfinite(ref)) and np.all(np.abs(r / ref - 1.0) <= 64 * EPS * yc.shape[1] ** 0.5)


_CASES = [
    (op, shape)
    for shape in ((512, 64, 1024), (300, 70, 520))  # one round of tiles; ragged (bounds, masked columns and rows)
    for op in ("max", "min", "sum", "product")
] + [("max", (4096, 128, 8192)), ("sum", (4096, 128, 8192))]  # 512 tiles: persistent workgroups


@pytest.mark.parametrize("op,shape", _CASES)
def test_fused_row_reduction(op, shape, monkeypatch):
    """Both forms -- row blocks combined across workgroups through the
    workspace, and row blocks walked whole by one workgroup -- on every
    shape (the assembler picks one by the number of row blocks; here each
    is forced); they combine in the same order, so they agree bit for bit."""
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", False)
    ref = run(_program(op, *shape), outputs=("Yc", "r", "z"))
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    got = {}
    for form in ("workspace", "local"):
        monkeypatch.setattr(mm, "rr_local", lambda *a, form=form, **k: form == "local")
        for attempt in range(2):  # the second launch finds the counters reset
            print(f"row-reduction epilogue: {op} {shape} {form} launch {attempt}", flush=True)
            res = run(_program(op, *shape), outputs=("Yc", "r", "z"))
            g = res.groups[0]
            assert g.strategy is FusionStrategy.MATMUL_REDUCTION_EPILOGUE and len(res.groups) == 2
            assert (g.kernel.workspace_bytes == 0) == (form == "local")
            np.testing.assert_array_equal(res.env["Yc"], ref.env["Yc"])
            np.testing.assert_array_equal(res.env["z"], ref.env["z"])
            _check_rows(op, res.env["r"], res.env["Yc"])
            if op in ("max", "min"):
                np.testing.assert_array_equal(res.env["r"], ref.env["r"])
            got.setdefault(form, res.env["r"])
            np.testing.assert_array_equal(res.env["r"], got[form])
    np.testing.assert_array_equal(got["local"], got["workspace"])
    # and against the oracle, at the matmul bar
    oracle = evaluate(_program(op, *shape))["r"]
    if op in ("max", "min"):
        np.testing.assert_allclose(got["local"], oracle, rtol=1e-4 * np.sqrt(shape[1]), atol=1e-5)


@pytest.mark.parametrize("form", ["workspace", "local", "k-resident"])
def test_attention_heads_batched(form, monkeypatch):
    """C5 at 512 x 64 for 6 heads in one batched launch per kernel: with the
    row max in the score kernel every output is the reference partition's
    (the LDS-tiled kernel in both of its forms, and the K-resident kernel)."""
    monkeypatch.setattr(mm, "K_RESIDENT", form == "k-resident")
    monkeypatch.setattr(mm, "rr_local", lambda *a, **k: form == "local")
    heads = 6
    make = lambda: [gpu_cases.attention_head(512, 64, head=h, heads=heads) for h in range(heads)]
    outs = ("Ss", "m1", "e", "s1", "O")
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", False)
    ref = run_batch(make(), outputs=outs)
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    for attempt in range(2):
        got = run_batch(make(), outputs=outs)
        assert len(got[0].groups) == 4 and got[0].groups[0].strategy is FusionStrategy.MATMUL_REDUCTION_EPILOGUE
        for h in range(heads):
            for name in outs:
                np.testing.assert_array_equal(got[h].env[name], ref[h].env[name], err_msg=f"head {h} {name}")


_SIZES = (33, 64, 100, 130, 256, 257, 512, 768)


@pytest.mark.parametrize("seed", range(24))
def test_random_matmul_row_reductions(seed, monkeypatch):
    """Seeded random shapes (aligned and ragged), reductions and lane-agnostic
    epilogues with the extension on: the matmul output is the reference
    partition's, and the row values are the reduction of that output."""
    rng = np.random.default_rng(1000 + seed)
    M, K, N = (int(rng.choice(_SIZES)) for _ in range(3))
    op = str(rng.choice(["max", "min", "sum", "product"]))
    epi = [str(e) for e in rng.choice(["scale", "negate", "relu", "shift"], size=int(rng.integers(0, 3)))]

    def program():
        r = np.random.default_rng(seed)
        ops = Operations()
        ops.from_numpy(r.standard_normal((M, K)).astype(np.float32), "A")
        ops.from_numpy((r.standard_normal((K, N)) / (4.0 * np.sqrt(K))).astype(np.float32), "B")
        ops.matmul(a="A", b="B", out="Y")
        cur = "Y"
        for i, e in enumerate(epi):
            nxt = f"E{i}"
            if e == "scale":
                ops.elementwise("mul", out=nxt, operands=(cur, 0.75))
            elif e == "negate":
                ops.elementwise("negate", out=nxt, operands=(cur,))
            elif e == "relu":
                ops.elementwise("max", out=nxt, operands=(cur, 0.0))
            else:
                ops.elementwise("add", out=nxt, operands=(cur, 1.0))
            cur = nxt
        if op == "product":  # values near 1 keep row products finite
            ops.elementwise("mul", out="Pm", operands=(cur, 0.05))
            ops.elementwise("add", out="Pa", operands=("Pm", 1.0))
            cur = "Pa"
        ops.reduction(op, out="r", x=cur)
        ops.elementwise("mul", out="z", operands=(cur, 2.0))  # the matmul output stays a program value
        return ops, cur

    print(f"random row reduction {seed}: {op} {(M, K, N)} epilogue {epi}", flush=True)
    ops_off, out = program()
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", False)
    ref = run(ops_off, outputs=(out, "r"))
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    res = run(program()[0], outputs=(out, "r"))
    assert res.groups[0].strategy is FusionStrategy.MATMUL_REDUCTION_EPILOGUE
    np.testing.assert_array_equal(res.env[out], ref.env[out])
    _check_rows(op, res.env["r"], res.env[out])
    if op in ("max", "min"):
        np.testing.assert_array_equal(res.env["r"], ref.env["r"])
