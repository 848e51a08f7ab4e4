"""The row-owning-wave matmul on the GPU against float64 products and
against the LDS-tiled kernel (``assembly.matmul.ROW_WAVES`` off): without a
prologue, with a row-divisor prologue in both of its k loops (plain divisors
and ones below 1, zero or subnormal), with a scalar prologue and a register
epilogue, and C5's batched attention heads.  The two kernels use different
MFMA shapes, so they agree to rounding, not bit for bit; each is
reproducible launch to launch."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run, run_batch
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly import matmul as mm
from tests import gpu_cases
from tests.matmul_check import check_matmul

pytestmark = pytest.mark.gpu


def _case(kind: str, M: int = 512, K: int = 2048):
    rng = np.random.default_rng(61)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, 128)).astype(np.float32)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    if kind == "plain":
        ops.matmul(a="A", b="B", out="Y")
        return ops, "Y", a, b
    if kind.startswith("divisor"):
        s = (rng.random(M) * 10.0 + 1.0).astype(np.float32)
        if kind == "divisor, per-element loop":
            s[[3, 260, 261]] = np.array([0.5, 0.0, 1e-40], dtype=np.float32)
        ops.from_numpy(s, "s")
        ops.reshape("s", (M, 1), out="sv")
        ops.elementwise("div", out="P", operands=("A", "sv"), y_broadcast="col")
        ops.matmul(a="P", b="B", out="Y")
        return ops, "Y", a / s[:, None], b
    ops.elementwise("mul", out="P", operands=("A", 0.25))  # scalar prologue, relu epilogue
    ops.matmul(a="P", b="B", out="Y0")
    ops.elementwise("max", out="Y", operands=("Y0", 0.0))
    return ops, "Y", a * np.float32(0.25), b


_KINDS = ["plain", "divisor, plain loop", "divisor, per-element loop", "scalar prologue, relu epilogue"]


@pytest.mark.parametrize("kind", _KINDS)
def test_row_waves_against_float64_and_the_lds_tiled_kernel(kind, monkeypatch):
    outs = {}
    for rows in (True, False):
        monkeypatch.setattr(mm, "ROW_WAVES", rows)
        ops, out, a, b = _case(kind)
        print(f"row waves: {kind} rows={rows}", flush=True)
        res = run(ops, outputs=(out,))
        body = res.groups[-1].kernel.source.split('extern "C"')[-1]
        assert ("mt_rw_chunk(" in body) == rows, kind
        outs[rows] = res.env[out]
    got, ref = outs[True], outs[False]
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-4, atol=1e-4)
    if kind == "divisor, per-element loop":
        good = np.all(np.isfinite(a), axis=1)  # rows with a finite A
        check_matmul(got[good], a[good], b, kind, a_rel=2.0 ** -22)
    elif kind == "scalar prologue, relu epilogue":
        # relu is 1-Lipschitz: the matmul bar holds for relu of the product
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        bound = 1e-4 * np.sqrt(a.shape[1]) * (np.abs(a64) @ np.abs(b64))
        assert np.all(np.abs(got - np.maximum(a64 @ b64, 0.0)) <= bound)
    else:
        check_matmul(got, a, b, kind, a_rel=2.0 ** -22 if kind.startswith("divisor") else 0.0)
    # reproducible launch to launch
    monkeypatch.setattr(mm, "ROW_WAVES", True)
    again = run(_case(kind)[0], outputs=(_case(kind)[1],)).env[_case(kind)[1]]
    np.testing.assert_array_equal(again, got)


def test_attention_heads_batched(monkeypatch):
    """C5 at 2048 x 128 for 4 heads in one batched launch: O against the
    float64 product of the kernel's own e / s1 and V, and against the
    LDS-tiled kernel; the other outputs unchanged bit for bit."""
    heads = 4
    outs = ("e", "s1", "O")
    make = lambda: [gpu_cases.attention_head(2048, 128, head=h, heads=heads) for h in range(heads)]
    got = {}
    for rows in (True, False):
        monkeypatch.setattr(mm, "ROW_WAVES", rows)
        print(f"row waves: attention heads rows={rows}", flush=True)
        res = run_batch(make(), outputs=outs)
        assert ("mt_rw_chunk(" in res[0].groups[-1].kernel.source.split('extern "C"')[-1]) == rows
        got[rows] = res
    for h in range(heads):
        e, s1 = got[True][h].env["e"], got[True][h].env["s1"]
        np.testing.assert_array_equal(e, got[False][h].env["e"])
        np.testing.assert_array_equal(s1, got[False][h].env["s1"])
        v = make()[h].uploads["V"]
        check_matmul(got[True][h].env["O"], e / s1.reshape(-1, 1), v, f"head {h} O", a_rel=2.0 ** -22)
        np.testing.assert_allclose(got[True][h].env["O"], got[False][h].env["O"], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("seed", range(12))
def test_random_row_wave_programs(seed):
    """Seeded random matmuls the row-owning-wave kernel takes: M of 256 -
    1024, K of 1024 - 2304, A prologues over one or two row operands (a
    divisor, plain or not, and a shift) or a scalar, and Lipschitz
    epilogues -- against the float64 product of the prologue's float32
    output, at the matmul bar."""
    rng = np.random.default_rng(7000 + seed)
    M, K = 256 * int(rng.integers(1, 5)), 128 * int(rng.integers(8, 19))
    pro = str(rng.choice(["none", "scalar", "divisor", "divisor and shift", "rough divisor"]))
    epi = str(rng.choice(["none", "relu", "scale"]))
    r = np.random.default_rng(seed)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = (r.standard_normal((K, 128)) / np.sqrt(K)).astype(np.float32)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ap, cur = a, "A"
    if pro == "scalar":
        ops.elementwise("mul", out="P", operands=("A", 1.5))
        ap, cur = a * np.float32(1.5), "P"
    elif pro != "none":
        s = (r.random(M) * 4.0 + 1.0).astype(np.float32)
        if pro == "rough divisor":
            s[r.choice(M, 3, replace=False)] = np.array([0.25, 1e-3, 3e-39], dtype=np.float32)
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
            with np.errstate(over="ignore"):
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
    print(f"random row waves {seed}: {(M, K)} prologue {pro} epilogue {epi}", flush=True)
    res = run(ops, outputs=(out,))
    assert "mt_rw_chunk(" in res.groups[-1].kernel.source.split('extern "C"')[-1]
    got = res.env[out].astype(np.float64)
    # a row whose prologue overflowed (a subnormal divisor) is non-finite
    # throughout before the epilogue (relu may map its NaNs to 0); its inf /
    # nan pattern depends on the summation order
    fin = np.isfinite(ap).all(axis=1)
    if epi != "relu":
        assert not np.isfinite(got[~fin]).any()
    a64, b64 = ap[fin].astype(np.float64), b.astype(np.float64)
    y = a64 @ b64
    ref = {"none": y, "relu": np.maximum(y, 0.0), "scale": -0.5 * y}[epi]
    bound = (1e-4 * np.sqrt(K) + 4e-7) * (np.abs(a64) @ np.abs(b64)) * (0.5 if epi == "scale" else 1.0) + 1e-30
    assert np.all(np.abs(got[fin] - ref) <= bound), float(np.max(np.abs(got[fin] - ref) / bound))
