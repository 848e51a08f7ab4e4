"""Program builders shared by the GPU parity tests and the benchmark.

Each builder returns an ``Operations`` with seeded inputs attached via
``from_numpy``; shapes are parameters so the same program runs at test
sizes and at the BASELINE.json sizes."""

from __future__ import annotations

import numpy as np

from metellus_amd.orchestrator import Operations


def sigmoid_chain(M: int, N: int, seed: int = 1) -> Operations:
    """C2: out = sigmoid(a*b + c) * d, sigmoid = recip(add(exp(negate(.)), 1))."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    for name in "abcd":
        ops.from_numpy(rng.standard_normal((M, N)).astype(np.float32), name)
    ops.elementwise("mul", out="t1", operands=("a", "b"))
    ops.elementwise("add", out="t2", operands=("t1", "c"))
    ops.elementwise("negate", out="n", operands=("t2",))
    ops.elementwise("exp", out="e", operands=("n",))
    ops.elementwise("add", out="p", operands=("e", 1.0))
    ops.elementwise("recip", out="s", operands=("p",))
    ops.elementwise("mul", out="out", operands=("s", "d"))
    return ops


def softmax(M: int, N: int, seed: int = 2) -> Operations:
    """C3: row softmax as max -> sub(COL) -> exp -> sum -> div(COL)."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, N)).astype(np.float32), "x")
    ops.reduction("max", out="m1", x="x")
    ops.reshape("m1", (M, 1), out="m")
    ops.elementwise("subtract", out="sh", operands=("x", "m"), y_broadcast="col")
    ops.elementwise("exp", out="e", operands=("sh",))
    ops.reduction("sum", out="s1", x="e")
    ops.reshape("s1", (M, 1), out="sv")
    ops.elementwise("div", out="p", operands=("e", "sv"), y_broadcast="col")
    return ops


def matmul_bias_relu(M: int, K: int, N: int, seed: int = 0) -> Operations:
    """C1: relu(A @ B + bias_row), values U[-1, 1]."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.uniform(-1, 1, (M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.uniform(-1, 1, (K, N)).astype(np.float32), "B")
    ops.from_numpy(rng.uniform(-1, 1, (N,)).astype(np.float32), "bias")
    ops.reshape("bias", (1, N), out="bias_row")
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("add", out="Cb", operands=("C", "bias_row"), y_broadcast="row")
    ops.elementwise("max", out="y", operands=("Cb", 0.0))
    return ops


def plain_matmul(M: int, K: int, N: int, seed: int = 0) -> Operations:
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.matmul(a="A", b="B", out="C")
    return ops


def mlp_block(M: int, D: int, H: int, seed: int = 3, diamond: bool = False) -> Operations:
    """C4: (silu(X@W1) * (X@W2)) @ W3 with std 1/sqrt(fan_in); the diamond
    variant stops at z = (X@W1) * (X@W2)."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy((rng.standard_normal((M, D)) / np.sqrt(M)).astype(np.float32), "X")
    ops.from_numpy((rng.standard_normal((D, H)) / np.sqrt(D)).astype(np.float32), "W1")
    ops.from_numpy((rng.standard_normal((D, H)) / np.sqrt(D)).astype(np.float32), "W2")
    if not diamond:
        ops.from_numpy((rng.standard_normal((H, D)) / np.sqrt(H)).astype(np.float32), "W3")
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="X", b="W2", out="h2")
    if diamond:
        ops.elementwise("mul", out="z", operands=("h1", "h2"))
        return ops
    ops.elementwise("negate", out="n", operands=("h1",))
    ops.elementwise("exp", out="e", operands=("n",))
    ops.elementwise("add", out="p", operands=("e", 1.0))
    ops.elementwise("recip", out="s", operands=("p",))
    ops.elementwise("mul", out="g", operands=("h1", "s"))
    ops.elementwise("mul", out="z", operands=("g", "h2"))
    ops.matmul(a="z", b="W3", out="out")
    return ops


_QKV_CACHE: dict = {}


def attention_qkv(S: int, Dh: int, seed: int = 4, heads: int = 1):
    """Q, K, V of shape (heads, S, Dh), N(0, 1), drawn in that order."""
    key = (S, Dh, seed, heads)
    if key not in _QKV_CACHE:
        rng = np.random.default_rng(seed)
        _QKV_CACHE.clear()
        _QKV_CACHE[key] = tuple(rng.standard_normal((heads, S, Dh)).astype(np.float32) for _ in range(3))
    return _QKV_CACHE[key]


def attention_head(S: int, Dh: int, seed: int = 4, head: int = 0, heads: int = 1) -> Operations:
    """C5 (one head): softmax((Q @ K^T) / sqrt(Dh)) @ V, K^T a stride view."""
    q, k, v = attention_qkv(S, Dh, seed, heads)
    ops = Operations()
    ops.from_numpy(np.ascontiguousarray(q[head]), "Q")
    ops.from_numpy(np.ascontiguousarray(k[head]), "K")
    ops.from_numpy(np.ascontiguousarray(v[head]), "V")
    ops.transpose("K", out="Kt")
    ops.matmul(a="Q", b="Kt", out="S")
    ops.elementwise("mul", out="Ss", operands=("S", float(1.0 / np.sqrt(Dh))))
    ops.reduction("max", out="m1", x="Ss")
    ops.reshape("m1", (S, 1), out="m")
    ops.elementwise("subtract", out="sh", operands=("Ss", "m"), y_broadcast="col")
    ops.elementwise("exp", out="e", operands=("sh",))
    ops.reduction("sum", out="s1", x="e")
    ops.reshape("s1", (S, 1), out="sv")
    ops.elementwise("div", out="P", operands=("e", "sv"), y_broadcast="col")
    ops.matmul(a="P", b="V", out="O")
    return ops
