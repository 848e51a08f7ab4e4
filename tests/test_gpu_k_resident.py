"""The K-resident row-wave matmul (``mt_kr_*``) on the GPU: against float64
products (both bounds of ``tests/matmul_check.py``) and against the
LDS-tiled kernel (``assembly.matmul.K_RESIDENT`` off), for K = 64 and 128,
with no prologue, a row-divisor prologue (divisors above and below 1, zero
and subnormal), a scalar prologue with a relu epilogue; batched heads
against the same programs run alone (another column split, the same sums:
bit for bit); the row-reduction epilogue form against the reference
partition (max / min bit for bit, sum / product within their order
bounds); seeded random programs.  The two kernels use different MFMA
shapes, so they agree to rounding, not bit for bit; each is reproducible
launch to launch."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run, run_batch
from metellus_amd.orchestrator import Operations, fusion
from metellus_amd.orchestrator.assembly import matmul as mm
from metellus_amd.orchestrator.kernel_group import FusionStrategy
from tests import gpu_cases
from tests.matmul_check import check_matmul

pytestmark = pytest.mark.gpu

EPS = np.finfo(np.float32).eps


def _case(kind: str, M: int = 512, K: int = 128, N: int = 1024, seed: int = 71):
    """(ops, output, A as the kernel sees it (float32), B) for B = Bs^T read
    along K."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K)).astype(np.float32)
    bs = rng.standard_normal((N, K)).astype(np.float32)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(bs, "Bs")
    ops.transpose("Bs", out="B")
    b = np.ascontiguousarray(bs.T)
    if kind == "plain":
        ops.matmul(a="A", b="B", out="Y")
        return ops, "Y", a, b
    if kind.startswith("divisor"):
        s = (rng.random(M) * 10.0 + 1.0).astype(np.float32)
        if kind == "divisor, rough":
            s[[3, 260, 261]] = np.array([0.5, 0.0, 1e-40], dtype=np.float32)
        ops.from_numpy(s, "s")
        ops.reshape("s", (M, 1), out="sv")
        ops.elementwise("div", out="P", operands=("A", "sv"), y_broadcast="col")
        ops.matmul(a="P", b="B", out="Y")
        with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
            return ops, "Y", a / s[:, None], b
    ops.elementwise("mul", out="P", operands=("A", 0.25))  # scalar prologue, relu epilogue
    ops.matmul(a="P", b="B", out="Y0")
    ops.elementwise("max", out="Y", operands=("Y0", 0.0))
    return ops, "Y", a * np.float32(0.25), b


_KINDS = ["plain", "divisor", "divisor, rough", "scalar prologue, relu epilogue"]


def _body(res) -> str:
    return res.groups[-1].kernel.source.split('extern "C"')[-1]


@pytest.mark.parametrize("K", [64, 128])
@pytest.mark.parametrize("kind", _KINDS)
def test_k_resident_against_float64_and_the_lds_tiled_kernel(kind, K, monkeypatch):
    outs = {}
    for on in (True, False):
        monkeypatch.setattr(mm, "K_RESIDENT", on)
        ops, out, a, b = _case(kind, K=K)
        print(f"k-resident: {kind} K={K} on={on}", flush=True)
        res = run(ops, outputs=(out,))
        assert ("mt_kr_chunk<" in _body(res)) == on, kind
        outs[on] = res.env[out]
    got, ref = outs[True], outs[False]
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-4, atol=1e-4)
    if kind == "divisor, rough":
        good = np.all(np.isfinite(a), axis=1)  # rows with a finite A
        check_matmul(got[good], a[good], b, kind, a_rel=2.0 ** -22)
    elif kind == "scalar prologue, relu epilogue":
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        bound = 1e-4 * np.sqrt(K) * (np.abs(a64) @ np.abs(b64))  # relu is 1-Lipschitz
        assert np.all(np.abs(got - np.maximum(a64 @ b64, 0.0)) <= bound)
    else:
        check_matmul(got, a, b, f"{kind} K={K}", a_rel=2.0 ** -22 if kind.startswith("divisor") else 0.0)
    monkeypatch.setattr(mm, "K_RESIDENT", True)
    ops, out, _, _ = _case(kind, K=K)
    np.testing.assert_array_equal(run(ops, outputs=(out,)).env[out], got)  # reproducible


def test_column_splits_sum_alike():
    """Attention scores for 4 heads batched (2 chunks per workgroup) and the
    same heads alone (1 chunk per workgroup): bit-identical, every element
    within both float64 bounds."""
    heads = 4
    make = lambda: [gpu_cases.attention_head(2048, 128, head=h, heads=heads) for h in range(heads)]
    print("k-resident: 4 heads batched against alone", flush=True)
    batched = run_batch(make(), outputs=("Ss",))
    assert batched[0].groups[0].grid == (8, 8, 1)
    scale = float(np.float32(1.0 / np.sqrt(128)))
    for h, ops in enumerate(make()):
        alone = run(ops, outputs=("Ss",))
        assert alone.groups[0].grid == (16, 8, 1)
        assert "mt_kr_chunk<128>(" in alone.groups[0].kernel.source.split('extern "C"')[-1]
        np.testing.assert_array_equal(batched[h].env["Ss"], alone.env["Ss"], err_msg=f"head {h}")
        q, k = ops.uploads["Q"], ops.uploads["K"]
        check_matmul(alone.env["Ss"], q, np.ascontiguousarray(k.T), f"head {h} Ss", scale=scale)


def _reduce_program(op: str, M: int = 512, K: int = 128, N: int = 1024, seed: int = 72) -> Operations:
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((N, K)).astype(np.float32), "Bs")
    ops.transpose("Bs", out="B")
    ops.matmul(a="A", b="B", out="Y")
    scale, shift = (0.5, 0.0) if op != "product" else (1.0 / (8.0 * K), 1.0)
    ops.elementwise("mul", out="Ys", operands=("Y", scale))
    ops.elementwise("add", out="Yc", operands=("Ys", shift))
    ops.reduction(op, out="r", x="Yc")
    ops.elementwise("mul", out="z", operands=("Yc", 2.0))  # another reader of Yc
    return ops


@pytest.mark.parametrize("op", ["max", "min", "sum", "product"])
@pytest.mark.parametrize("K", [64, 128])
def test_row_reduction_epilogue(op, K, monkeypatch):
    """The matmul -> reduction extension on the K-resident kernel: the matmul
    output is the reference partition's bit for bit, and the row values are
    the reduction of exactly that output (max / min exact; sum / product
    within a fixed tree's bound), again on a second launch."""
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", False)
    ref = run(_reduce_program(op, K=K), outputs=("Yc", "r", "z"))
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    first = None
    for attempt in range(2):
        print(f"k-resident row reduction: {op} K={K} launch {attempt}", flush=True)
        res = run(_reduce_program(op, K=K), outputs=("Yc", "r", "z"))
        g = res.groups[0]
        assert g.strategy is FusionStrategy.MATMUL_REDUCTION_EPILOGUE and len(res.groups) == 2
        assert "mt_kr_chunk<" in g.kernel.source.split('extern "C"')[-1] and g.kernel.workspace_bytes == 0
        yc, r = res.env["Yc"], res.env["r"]
        np.testing.assert_array_equal(yc, ref.env["Yc"])
        np.testing.assert_array_equal(res.env["z"], ref.env["z"])
        if op in ("max", "min"):
            np.testing.assert_array_equal(r, getattr(yc, op)(axis=1))
            np.testing.assert_array_equal(r, ref.env["r"])
        elif op == "sum":
            exact = yc.astype(np.float64).sum(axis=1)
            bound = 64 * EPS * np.abs(yc).astype(np.float64).sum(axis=1)
            assert np.all(np.abs(r - exact) <= bound), np.max(np.abs(r - exact) / bound)
        else:
            exact = np.prod(yc.astype(np.float64), axis=1)
            assert np.all(np.isfinite(exact)) and np.all(np.abs(r / exact - 1.0) <= 64 * EPS * yc.shape[1] ** 0.5)
        if first is None:
            first = r
        np.testing.assert_array_equal(r, first)


def test_attention_heads_with_row_max(monkeypatch):
    """C5 at 2048 x 128 for 4 heads, batched: with the row max in the
    K-resident score kernel every output equals the reference partition's."""
    heads = 4
    make = lambda: [gpu_cases.attention_head(2048, 128, head=h, heads=heads) for h in range(heads)]
    outs = ("Ss", "m1", "e", "s1", "O")
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", False)
    print("k-resident: attention heads, reference partition", flush=True)
    ref = run_batch(make(), outputs=outs)
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    print("k-resident: attention heads, row max fused", flush=True)
    got = run_batch(make(), outputs=outs)
    assert len(got[0].groups) == 4 and got[0].groups[0].grid == (1, 8, 1)
    for h in range(heads):
        for name in outs:
            np.testing.assert_array_equal(got[h].env[name], ref[h].env[name], err_msg=f"head {h} {name}")


@pytest.mark.parametrize("seed", range(10))
def test_random_k_resident_programs(seed):
    """Seeded random matmuls the K-resident kernel takes: M of 256 - 1024,
    K of 64 or 128, N of 512 - 2048, A prologues over a row operand or a
    scalar, Lipschitz epilogues -- against float64 at the matmul bar."""
    rng = np.random.default_rng(8000 + seed)
    M, K, N = 256 * int(rng.integers(1, 5)), int(rng.choice([64, 128])), 128 * int(rng.integers(4, 17))
    pro = str(rng.choice(["none", "scalar", "divisor", "divisor and shift"]))
    epi = str(rng.choice(["none", "relu", "scale"]))
    r = np.random.default_rng(seed)
    a = r.standard_normal((M, K)).astype(np.float32)
    bs = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(bs, "Bs")
    ops.transpose("Bs", out="B")
    ap, cur = a, "A"
    if pro == "scalar":
        ops.elementwise("mul", out="P", operands=("A", 1.5))
        ap, cur = a * np.float32(1.5), "P"
    elif pro != "none":
        s = (r.random(M) * 4.0 + 0.5).astype(np.float32)
        ops.from_numpy(s, "s")
        ops.reshape("s", (M, 1), out="sv")
        if pro == "divisor and shift":
            t = r.standard_normal(M).astype(np.float32)
            ops.from_numpy(t, "t")
            ops.reshape("t", (M, 1), out="tv")
            ops.elementwise("subtract", out="Q", operands=("A", "tv"), y_broadcast="col")
            ops.elementwise("div", out="P", operands=("Q", "sv"), y_broadcast="col")
            ap = (a - t[:, None]) / s[:, None]
        else:
            ops.elementwise("div", out="P", operands=("A", "sv"), y_broadcast="col")
            ap = a / s[:, None]
        cur = "P"
    ops.matmul(a=cur, b="B", out="Y")
    out = "Y"
    if epi == "relu":
        ops.elementwise("max", out="Z", operands=("Y", 0.0))
        out = "Z"
    elif epi == "scale":
        ops.elementwise("mul", out="Z", operands=("Y", -0.5))
        out = "Z"
    print(f"random k-resident {seed}: {(M, K, N)} prologue {pro} epilogue {epi}", flush=True)
    res = run(ops, outputs=(out,))
    assert "mt_kr_chunk<" in _body(res)
    got = res.env[out].astype(np.float64)
    a64, b64 = ap.astype(np.float64), bs.T.astype(np.float64)
    y = a64 @ b64
    ref = {"none": y, "relu": np.maximum(y, 0.0), "scale": -0.5 * y}[epi]
    bound = (1e-4 * np.sqrt(K) + 4e-7) * (np.abs(a64) @ np.abs(b64)) * (0.5 if epi == "scale" else 1.0) + 1e-30
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))


@pytest.mark.parametrize("axis", ["col", "row"])
def test_epilogue_with_a_broadcast_operand(axis, monkeypatch):
    """Y = A @ B^T + bias with the bias per output column (a row vector) or
    per output row (a column vector): the K-resident epilogue reads it by the
    (row, col) each stored element has -- against the float64 product plus
    the bias, at the matmul bar, and against the LDS-tiled kernel."""
    M, K, N = 512, 128, 1024
    rng = np.random.default_rng(73)
    a = rng.standard_normal((M, K)).astype(np.float32)
    bs = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(N if axis == "col" else M).astype(np.float32)

    def program():
        ops = Operations()
        ops.from_numpy(a, "A")
        ops.from_numpy(bs, "Bs")
        ops.transpose("Bs", out="B")
        ops.from_numpy(bias, "bias")
        if axis == "col":
            ops.reshape("bias", (1, N), out="bv")
            bc = "row"  # one value per column, broadcast over the rows
        else:
            ops.reshape("bias", (M, 1), out="bv")
            bc = "col"
        ops.matmul(a="A", b="B", out="Y0")
        ops.elementwise("add", out="Y", operands=("Y0", "bv"), y_broadcast=bc)
        return ops

    got = {}
    for on in (True, False):
        monkeypatch.setattr(mm, "K_RESIDENT", on)
        print(f"k-resident: bias per {axis}, on={on}", flush=True)
        res = run(program(), outputs=("Y",))
        assert len(res.groups) == 1 and ("mt_kr_chunk<" in _body(res)) == on
        got[on] = res.env["Y"]
    y64 = a.astype(np.float64) @ bs.T.astype(np.float64)
    y64 = y64 + (bias[None, :] if axis == "col" else bias[:, None])
    mag = np.abs(a).astype(np.float64) @ np.abs(bs.T).astype(np.float64) + np.abs(y64)
    bound = (1e-4 * np.sqrt(K)) * mag + 1e-30
    assert np.all(np.abs(got[True] - y64) <= bound)
    np.testing.assert_allclose(got[True], got[False], rtol=1e-4, atol=1e-4)
