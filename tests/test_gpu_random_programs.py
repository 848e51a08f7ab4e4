"""Seeded random programs through ``api.run`` on the GPU, against the CPU
oracle -- a differential sweep over the launch-shape decisions the fixed
tests pin at a few sizes (direct-to-LDS vs register loads, 16- vs 8-wave
tiles, persistent and stream-K loops, bounds-checked edges, transposed
views, prologue / epilogue fusion, diamonds, reductions).

Bars, derived per program:

* elementwise chains of IEEE-exact ops: exact (NaN == NaN);
* reductions over an exact prologue: max / min exact, sum bit-identical to
  the replay of the kernel's combine order, a scalar epilogue exact on top;
* matmuls: |err| <= L * (1e-4 sqrt(K) (|A'| @ |B'|) + 4 u (|A'| @ |B'|))
  where A', B' are the operands after their prologues (the 4 u covers the
  matmul loaders' fast division, within 2 ulp) and L bounds how much the
  epilogue chain can magnify an error (|c| for a scalar multiply, 1 for
  add / max / negate), plus 2 u |result| for each epilogue rounding;
* diamonds: the product / sum / max bounds of the two anchors' bars.
"""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import compile_program, run
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly.reduction import reduction_order
from metellus_amd.orchestrator.ir import ReductionOp
from oracle.ir_eval import evaluate, ordered_row_reduce

pytestmark = pytest.mark.gpu

U = 2.0**-24
ALIGNED = (256, 512, 768, 1024)
RAGGED = (33, 64, 96, 100, 130, 200, 257)


def _f32(rng, shape, lo=-2.0, hi=2.0):
    return rng.uniform(lo, hi, shape).astype(np.float32)


def _dim(rng, aligned_p=0.6):
    pool = ALIGNED if rng.random() < aligned_p else RAGGED
    return int(rng.choice(pool))


def _bar(a, b):
    a64, b64 = np.abs(a.astype(np.float64)), np.abs(b.astype(np.float64))
    m = a64 @ b64
    return (1e-4 * np.sqrt(a.shape[1]) + 4 * U) * m


# ---------------------------------------------------------------------------
# program families: each returns (ops, check(env))
# ---------------------------------------------------------------------------


def matmul_program(rng):
    M, K, N = _dim(rng), _dim(rng), _dim(rng)
    ops = Operations()
    x = _f32(rng, (M, K))
    if rng.random() < 0.3:  # A as a transposed view of a stored (K, M)
        ops.from_numpy(np.ascontiguousarray(x.T), "Xs")
        ops.transpose("Xs", out="A")
    else:
        ops.from_numpy(x, "A")
    w = _f32(rng, (K, N))
    if rng.random() < 0.3:  # B as a transposed view (K^T-like)
        ops.from_numpy(np.ascontiguousarray(w.T), "Ws")
        ops.transpose("Ws", out="B")
    else:
        ops.from_numpy(w, "B")
    a_name, a_val = "A", x
    kind = rng.integers(0, 5)
    if kind == 1:
        ops.elementwise("mul", out="Ap", operands=("A", 0.5))
        a_name, a_val = "Ap", x * np.float32(0.5)
    elif kind == 2:
        y = _f32(rng, (M, K))
        ops.from_numpy(y, "Y")
        ops.elementwise("add", out="Ap", operands=("A", "Y"))
        a_name, a_val = "Ap", x + y
    elif kind == 3:
        ops.elementwise("max", out="Ap", operands=("A", 0.0))
        a_name, a_val = "Ap", np.maximum(x, np.float32(0.0))
    elif kind == 4:
        d = _f32(rng, (M,), 1.0, 2.0)
        ops.from_numpy(d, "d")
        ops.reshape("d", (M, 1), out="dc")
        ops.elementwise("div", out="Ap", operands=("A", "dc"), y_broadcast="col")
        a_name, a_val = "Ap", x / d[:, None]
    ops.matmul(a=a_name, b="B", out="C")
    out, L, roundings = "C", 1.0, 0
    for step in range(int(rng.integers(0, 3))):
        e = int(rng.integers(0, 4))
        nxt = f"E{step}"
        if e == 0:
            bias = _f32(rng, (N,))
            ops.from_numpy(bias, f"bias{step}")
            ops.reshape(f"bias{step}", (1, N), out=f"brow{step}")
            ops.elementwise("add", out=nxt, operands=(out, f"brow{step}"), y_broadcast="row")
        elif e == 1:
            ops.elementwise("mul", out=nxt, operands=(out, -1.5))
            L *= 1.5
        elif e == 2:
            ops.elementwise("max", out=nxt, operands=(out, 0.0))
        else:
            ops.elementwise("negate", out=nxt, operands=(out,))
        roundings += 1
        out = nxt

    def check(env):
        ref = evaluate(ops)[out].astype(np.float64)
        bar = L * _bar(a_val, w) + (2 * roundings + 1) * U * np.abs(ref) + 1e-30
        err = np.abs(env[out].astype(np.float64) - ref)
        assert np.all(err <= bar), f"{(M, K, N)}: max err/bar {np.max(err / bar):.3f}"

    return ops, out, check


def elementwise_program(rng):
    M, N = _dim(rng, 0.4), _dim(rng, 0.4)
    n_in = int(rng.integers(1, 4))
    plan = []  # (op, other input index) -- planned first so only used tensors are uploaded
    for _ in range(int(rng.integers(2, 6))):
        plan.append((int(rng.integers(0, 9)), int(rng.integers(0, n_in))))
    used = {0} | {j for k, j in plan if k in (0, 3, 7, 8)}
    ops = Operations()
    for i in sorted(used):
        ops.from_numpy(_f32(rng, (M, N), -3, 3), f"x{i}")
    if any(k == 1 for k, _ in plan):
        ops.from_numpy(_f32(rng, (N,), -3, 3), "r")
        ops.reshape("r", (1, N), out="rr")
    if any(k == 2 for k, _ in plan):
        ops.from_numpy(_f32(rng, (M,), 0.5, 3), "c")
        ops.reshape("c", (M, 1), out="cc")
    cur = "x0"
    for step, (k, j) in enumerate(plan):
        nxt, other = f"t{step}", f"x{j}"
        if k == 0:
            ops.elementwise("add", out=nxt, operands=(cur, other))
        elif k == 1:
            ops.elementwise("mul", out=nxt, operands=(cur, "rr"), y_broadcast="row")
        elif k == 2:
            ops.elementwise("div", out=nxt, operands=(cur, "cc"), y_broadcast="col")
        elif k == 3:
            ops.elementwise("max", out=nxt, operands=(cur, other))
        elif k == 4:
            ops.elementwise("subtract", out=nxt, operands=(cur, 0.75))
        elif k == 5:
            ops.elementwise("absolute", out=nxt, operands=(cur,))
        elif k == 6:
            ops.elementwise("floor", out=nxt, operands=(cur,))
        elif k == 7:
            ops.elementwise("gt", out=nxt, operands=(cur, other))
        else:
            ops.elementwise("where", out=nxt, operands=(cur, other, "x0"))
        cur = nxt

    def check(env):
        np.testing.assert_array_equal(env[cur], evaluate(ops)[cur])

    return ops, cur, check


def reduction_program(rng):
    M, N = _dim(rng, 0.4), int(rng.choice((64, 100, 256, 1000, 2048, 4099)))
    ops = Operations()
    x = _f32(rng, (M, N), -3, 3)
    ops.from_numpy(x, "x")
    src = "x"
    if rng.random() < 0.5:
        y = _f32(rng, (M, N), -3, 3)
        ops.from_numpy(y, "y")
        ops.elementwise("mul", out="xp", operands=("x", "y"))
        src = "xp"
    op = str(rng.choice(["sum", "max", "min"]))
    ops.reduction(op, out="r", x=src)
    out = "r"
    if rng.random() < 0.5:
        ops.elementwise("mul", out="rs", operands=("r", 0.25))
        out = "rs"

    def check(env):
        ref = evaluate(ops)
        if op == "sum":
            g = next(g for g in compile_program(ops) if any(isinstance(o, ReductionOp) for o in g.ops))
            o = reduction_order(g)
            vals = x if src == "x" else ref["xp"]
            r = ordered_row_reduce(vals, "sum", o["waves_per_row"], o["vectorized"])
            expect = r if out == "r" else (r * np.float32(0.25)).astype(np.float32)
        else:
            expect = ref[out]
        np.testing.assert_array_equal(env[out], expect)

    return ops, out, check


def diamond_program(rng):
    M, K, N = _dim(rng), _dim(rng), _dim(rng)
    ops = Operations()
    x, w1, w2 = _f32(rng, (M, K)), _f32(rng, (K, N)), _f32(rng, (K, N))
    ops.from_numpy(x, "X")
    ops.from_numpy(w1, "W1")
    ops.from_numpy(w2, "W2")
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="X", b="W2", out="h2")
    merge = str(rng.choice(["mul", "add", "max", "subtract"]))
    ops.elementwise(merge, out="z", operands=("h1", "h2"))

    def check(env):
        x64 = x.astype(np.float64)
        h1, h2 = x64 @ w1.astype(np.float64), x64 @ w2.astype(np.float64)
        t1, t2 = _bar(x, w1), _bar(x, w2)
        if merge == "mul":
            ref, bound = h1 * h2, np.abs(h2) * t1 + np.abs(h1) * t2 + t1 * t2
        elif merge == "add":
            ref, bound = h1 + h2, t1 + t2
        elif merge == "subtract":
            ref, bound = h1 - h2, t1 + t2
        else:
            ref, bound = np.maximum(h1, h2), np.maximum(t1, t2)
        bound = bound + 2 * U * np.abs(ref) + 1e-30
        err = np.abs(env["z"].astype(np.float64) - ref)
        assert np.all(err <= bound), f"{(M, K, N)} {merge}: max err/bar {np.max(err / bound):.3f}"

    return ops, "z", check


FAMILIES = (
    [("matmul", matmul_program, s) for s in range(56)]
    + [("elementwise", elementwise_program, s) for s in range(30)]
    + [("reduction", reduction_program, s) for s in range(24)]
    + [("diamond", diamond_program, s) for s in range(16)]
)


@pytest.mark.parametrize("family,make,seed", FAMILIES, ids=[f"{f}-{s}" for f, _, s in FAMILIES])
def test_random_program(family, make, seed):
    rng = np.random.default_rng(1000 + seed * 7 + len(family))
    ops, out, check = make(rng)
    res = run(ops, outputs=(out,))
    check(res.env)


@pytest.mark.parametrize("seed", range(24))
def test_random_program_persistent(seed, monkeypatch):
    """Matmuls and diamonds with a small resident capacity, so their tiles
    take the persistent loop and, for partial last rounds, stream-K."""
    from metellus_amd.compute.matmul import config

    rng = np.random.default_rng(5000 + seed)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", int(rng.choice((3, 5, 7, 13))))
    make = matmul_program if seed % 3 else diamond_program
    ops, out, check = make(rng)
    res = run(ops, outputs=(out,))
    check(res.env)
    from metellus_amd.runtime import hip_backend

    hip_backend.check_workspace()
