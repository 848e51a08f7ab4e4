"""GPU parity at the benchmark configurations' full sizes (C1 256^3 is
covered by ``test_gpu_parity.test_c1_matmul_bias_relu`` at its own size).

Each kernel is checked against the oracle fed with the *GPU's own* inputs
to that kernel (the downloaded intermediates), so every bar is the
per-kernel bar and errors do not compound across kernels:

* IEEE-exact kernels (max reductions, divisions, products of operands):
  exact equality;
* sum reductions: bit-identical to the oracle's replay of the kernel's
  combine order (``ordered_row_reduce``);
* chains with ``exp``: rtol = atol = 1e-5 (the two sides use different
  ``exp`` implementations);
* matmuls: every element of the output against the float64 product of the
  same float32 operands, within the stated bar 1e-4 * sqrt(K) * (|A| @ |B|)
  and within the float32 accumulation bound 2 gamma_K (|A| @ |B|)
  (``tests/matmul_check.py``), which a dropped or duplicated k-chunk of any
  tile -- data-parallel, persistent or stream-K -- exceeds.

Size-independent properties on top: softmax rows sum to 1 within the
float32 accumulation bound of the kernel's combine order, and end-to-end
attention rows against float64 attention.
"""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import compile_program, run, run_batch
from metellus_amd.orchestrator.assembly.reduction import reduction_order
from oracle.ir_eval import apply_elementwise, evaluate, ordered_row_reduce
from tests import gpu_cases
from tests.matmul_check import check_matmul, check_matmul_product

pytestmark = pytest.mark.gpu

U32 = 2.0**-24  # unit roundoff of float32


def _order(ops, name: str) -> dict:
    g = next(g for g in compile_program(ops) if g.kernel.function_name == f"reduce_{name}_fused")
    return reduction_order(g)


def test_c2_sigmoid_chain_4096():
    """C2: out = sigmoid(a*b + c) * d on 4 x 4096x4096, whole output."""
    ops = gpu_cases.sigmoid_chain(4096, 4096, seed=1)
    res = run(ops, outputs=("out",))
    assert len(res.groups) == 1
    np.testing.assert_allclose(res.env["out"], evaluate(ops)["out"], rtol=1e-5, atol=1e-5)


def test_c3_softmax_8192():
    """C3: softmax of 8192x8192, every kernel on the whole matrix."""
    ops = gpu_cases.softmax(8192, 8192, seed=2)
    res = run(ops)
    assert len(res.groups) == 4
    x = ops.uploads["x"]
    env = res.env
    # K1 row max: exact
    np.testing.assert_array_equal(env["m1"], np.fmax.reduce(x, axis=1))
    # K2 e = exp(x - m) on the GPU's m1 (x - m is exact)
    e_ref = apply_elementwise("exp", apply_elementwise("subtract", x, env["m1"][:, None]))
    np.testing.assert_allclose(env["e"], e_ref, rtol=1e-5, atol=1e-5)
    # K3 row sum: bit-identical to the replay of the kernel's order
    o = _order(ops, "s1")
    np.testing.assert_array_equal(env["s1"], ordered_row_reduce(env["e"], "sum", o["waves_per_row"], o["vectorized"]))
    # K4 p = e / s: IEEE division, exact
    np.testing.assert_array_equal(env["p"], env["e"] / env["s1"][:, None])
    # property: rows sum to 1.  The kernel's sum is a sequence of at most
    # 8192/256 per-lane adds, 2 + 6 tree levels, so |s1 - sum e| <= 40 u sum e;
    # each quotient adds u.
    dev = np.abs(env["p"].astype(np.float64).sum(axis=1) - 1.0)
    assert dev.max() <= 42 * U32 * 1.01, dev.max()


def test_matmul_4096_cubed():
    """4096^3: every output element against float64."""
    ops = gpu_cases.plain_matmul(4096, 4096, 4096, seed=0)
    res = run(ops)
    print("4096^3: checking the whole output against float64", flush=True)
    check_matmul(res.env["C"], ops.uploads["A"], ops.uploads["B"], "4096^3 C")


def test_c4_mlp_block_literal_full():
    """C4 literal: X@W1, X@W2 (stream-K persistent), the sigmoid chain, and
    (h1*s*h2)@W3 with the chain in the A loader -- each kernel's whole
    output against its own GPU inputs."""
    ops = gpu_cases.mlp_block(4096, 4096, 11008, seed=3)
    res = run(ops)
    assert len(res.groups) == 4
    env = res.env
    for h, w in (("h1", "W1"), ("h2", "W2")):
        print(f"C4 {h}: checking the whole output against float64", flush=True)
        check_matmul(env[h], ops.uploads["X"], ops.uploads[w], f"C4 {h}")
    h1 = env["h1"]
    s_ref = h1
    for op, arg in (("negate", None), ("exp", None), ("add", np.float32(1.0)), ("recip", None)):
        s_ref = apply_elementwise(op, s_ref, arg)
    np.testing.assert_allclose(env["s"], s_ref, rtol=1e-5, atol=1e-5)
    del s_ref
    # prologue g = h1 * s, z = g * h2, each one IEEE multiply: the kernel's A operand exactly
    z = apply_elementwise("mul", apply_elementwise("mul", h1, env["s"]), env["h2"])
    print("C4 out: checking the whole output against float64", flush=True)
    check_matmul(env["out"], z, ops.uploads["W3"], "C4 out")


def test_c4_diamond_full():
    """(X@W1) * (X@W2) in one kernel at 4096 x 4096 x 11008 (1376 tiles,
    stream-K last round handing over both accumulator sets): whole output."""
    ops = gpu_cases.mlp_block(4096, 4096, 11008, seed=3, diamond=True)
    res = run(ops)
    assert len(res.groups) == 1
    print("C4 diamond: checking the whole output against float64", flush=True)
    check_matmul_product(res.env["z"], ops.uploads["X"], ops.uploads["W1"], ops.uploads["W2"], "C4 diamond z")


def test_c5_attention_32_heads_full():
    """C5: 32 heads x 2048 x 128, one batched launch per kernel.  Exact and
    replayed kernels, and both matmuls whole, on every head; end-to-end
    attention rows of every head against float64."""
    heads, S, Dh = 32, 2048, 128
    progs = [gpu_cases.attention_head(S, Dh, seed=4, head=h, heads=heads) for h in range(heads)]
    results = run_batch(progs)
    o = _order(progs[0], "s1")
    scale = np.float32(1.0 / np.sqrt(Dh))
    rng = np.random.default_rng(10)
    for h, (ops, res) in enumerate(zip(progs, results)):
        env = res.env
        assert "P" not in env  # e / s is the P@V kernel's prologue
        ss = env["Ss"]
        np.testing.assert_array_equal(env["m1"], np.fmax.reduce(ss, axis=1), err_msg=f"head {h} m1")
        e_ref = apply_elementwise("exp", apply_elementwise("subtract", ss, env["m1"][:, None]))
        np.testing.assert_allclose(env["e"], e_ref, rtol=1e-5, atol=1e-5, err_msg=f"head {h} e")
        np.testing.assert_array_equal(
            env["s1"], ordered_row_reduce(env["e"], "sum", o["waves_per_row"], o["vectorized"]), err_msg=f"head {h} s1"
        )
        q, k, v = (ops.uploads[n] for n in "QKV")
        check_matmul(ss, q, np.ascontiguousarray(k.T), f"head {h} Ss", scale=float(scale))
        # the P@V loader's division is within 2 ulp (4u relative) of IEEE's
        check_matmul(env["O"], env["e"] / env["s1"][:, None], v, f"head {h} O", a_rel=4 * U32)
        q, k, v = (x.astype(np.float64) for x in (q, k, v))
        rows = rng.choice(S, 16, replace=False)
        logits = (q[rows] @ k.T) * float(scale)
        pr = np.exp(logits - logits.max(axis=1, keepdims=True))
        pr /= pr.sum(axis=1, keepdims=True)
        np.testing.assert_allclose(env["O"][rows], pr @ v, rtol=1e-3, atol=1e-4, err_msg=f"head {h} O rows")
