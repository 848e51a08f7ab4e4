"""CPU oracle for the Metellus fused-kernel path (test infrastructure only).

This module is the *checker* for the HIP backend: tests, ``smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; product code never does
(the product path fails loudly without its HIP library instead of falling
back here).

It restates, in NumPy, what the reference's generated kernels compute for a
program built with ``Operations`` -- the IR semantics, independent of how
the program is fused:

* elementwise ops -- the reference op table (reference:
  src/compute/elementwise/elementwise.py:18-58) evaluated in float32, one
  correctly rounded operation at a time (``-ffp-contract=off`` on the GPU
  side); ``max``/``min`` are ``fmax``/``fmin`` (a NaN operand loses),
  ``sign(NaN) = 0``, ``tanh`` is the saturating form, comparisons give
  1.0/0.0, ``where(x, y, cond) = cond != 0 ? x : y``; Scalars are fp32
  literals (reference: src/orchestrator/assembly/expressions.py:51-57);
* broadcasts NONE/SCALAR/ROW/COL (reference: src/orchestrator/ir.py:262-308);
* tensors are strided views of their storage owner's buffer
  (``buffer_key``), so transposes / reshape views read what the kernels
  read (reference: src/orchestrator/ir.py:53-246);
* last-axis reductions with identities sum 0, product 1, max -inf, min +inf
  (reference: src/compute/reduction/reduction.py:172-193);
* matmul accumulated in float64 (the reference for a tolerance check);
* ``ShapeOp`` -- a strided gather (reference: src/compute/copy/copy.py:25-54).

``ordered_row_reduce`` additionally replays the exact combine order of the
gfx950 reduction kernel (lane chunks, four vector accumulators, wave64
butterfly, cross-wave fold), so sums and products can be compared bit for
bit.  How each function is pinned (known-answer vectors, closed forms,
invariants) is listed in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# ---------------------------------------------------------------------------
# elementwise semantics
# ---------------------------------------------------------------------------


def _tanh(x):
    # copysign(1 - 2/(1 + exp(2|x|)), x), each step in float32
    with np.errstate(over="ignore"):
        t = np.exp(F32(2.0) * np.abs(x))
    r = F32(1.0) - F32(2.0) / (F32(1.0) + t)
    return np.copysign(r, x).astype(F32)


def _sign(x):
    return np.where(x > 0, F32(1.0), np.where(x < 0, F32(-1.0), F32(0.0))).astype(F32)


UNARY = {
    "negate": lambda x: -x,
    "absolute": np.abs,
    "exp": np.exp,
    "log": np.log,
    "sqrt": np.sqrt,
    "recip": lambda x: F32(1.0) / x,
    "sin": np.sin,
    "cos": np.cos,
    "tanh": _tanh,
    "floor": np.floor,
    "ceil": np.ceil,
    "sign": _sign,
}

BINARY = {
    "add": lambda x, y: x + y,
    "subtract": lambda x, y: x - y,
    "mul": lambda x, y: x * y,
    "div": lambda x, y: x / y,
    "max": np.fmax,
    "min": np.fmin,
    "pow": np.power,
    "equal": lambda x, y: (x == y).astype(F32),
    "not_equal": lambda x, y: (x != y).astype(F32),
    "lt": lambda x, y: (x < y).astype(F32),
    "gt": lambda x, y: (x > y).astype(F32),
    "ge": lambda x, y: (x >= y).astype(F32),
    "le": lambda x, y: (x <= y).astype(F32),
}


def apply_elementwise(op: str, x, y=None, cond=None):
    """One elementwise op in float32 (inputs already broadcast)."""
    with np.errstate(all="ignore"):
        if op in UNARY:
            return np.asarray(UNARY[op](x), dtype=F32)
        if op in BINARY:
            return np.asarray(BINARY[op](x, y), dtype=F32)
        if op == "where":
            return np.where(cond != F32(0.0), x, y).astype(F32)
    raise ValueError(f"unknown elementwise op {op!r}")


REDUCE_IDENTITY = {"sum": 0.0, "product": 1.0, "max": -np.inf, "min": np.inf}


def reduce_rows(x, op: str):
    """Reference semantics of a last-axis reduction (order-free check).
    sum/product accumulate in float64; max/min ignore NaN like fmaxf/fminf."""
    with np.errstate(all="ignore"):
        if op == "sum":
            return x.astype(np.float64).sum(axis=-1)
        if op == "product":
            return x.astype(np.float64).prod(axis=-1)
        if op == "max":
            return np.fmax.reduce(x, axis=-1).astype(F32)
        if op == "min":
            return np.fmin.reduce(x, axis=-1).astype(F32)
    raise ValueError(f"unknown reduction op {op!r}")


# ---------------------------------------------------------------------------
# exact replay of the gfx950 reduction order
# ---------------------------------------------------------------------------


def _combine(op: str):
    return {
        "sum": lambda a, b: a + b,
        "product": lambda a, b: a * b,
        "max": np.fmax,
        "min": np.fmin,
    }[op]


def ordered_row_reduce(x, op: str, waves_per_row: int, vectorized: bool):
    """Replay the kernel's combine order in float32 for every row of ``x``
    (values already prologue-transformed):

    lanes t < T = 64*W; vector path: lane t folds float4 chunks q = t, t+T,
    ... into a_j (element 4q+j), lane value (a0 op a1) op (a2 op a3); scalar
    path: lane t folds elements t, t+T, ... into a0.  Then per wave the
    butterfly v = v op v[l ^ off], off = 32..1; then waves fold left to
    right.  Returns float32 of shape (rows,)."""
    x = np.asarray(x, dtype=F32)
    rows, K = x.shape
    comb = _combine(op)
    ident = F32(REDUCE_IDENTITY[op])
    T = 64 * waves_per_row
    with np.errstate(all="ignore"):
        if vectorized:
            assert K % 4 == 0
            nq = K // 4
            chunks = x.reshape(rows, nq, 4)
            acc = np.full((rows, T, 4), ident, dtype=F32)
            for start in range(0, nq, T):
                q = np.arange(start, min(start + T, nq))
                lanes = q - start
                acc[:, lanes, :] = comb(acc[:, lanes, :], chunks[:, q, :])
            lane_v = comb(comb(acc[:, :, 0], acc[:, :, 1]), comb(acc[:, :, 2], acc[:, :, 3]))
        else:
            acc = np.full((rows, T), ident, dtype=F32)
            for start in range(0, K, T):
                e = np.arange(start, min(start + T, K))
                lanes = e - start
                acc[:, lanes] = comb(acc[:, lanes], x[:, e])
            lane_v = acc
        lane_v = lane_v.astype(F32).reshape(rows, waves_per_row, 64)
        idx = np.arange(64)
        for off in (32, 16, 8, 4, 2, 1):
            lane_v = comb(lane_v, lane_v[:, :, idx ^ off]).astype(F32)
        r = lane_v[:, 0, 0]
        for w in range(1, waves_per_row):
            r = comb(r, lane_v[:, w, 0]).astype(F32)
    return np.asarray(r, dtype=F32)


# ---------------------------------------------------------------------------
# program evaluation
# ---------------------------------------------------------------------------


def _view(storage: np.ndarray, t) -> np.ndarray:
    """Read tensor ``t`` out of its owner's flat storage via its strides."""
    flat = storage.reshape(-1)
    item = flat.itemsize
    if len(t.shape) == 0:
        return flat[:1].reshape(())
    if len(t.shape) == 1:
        strides = (t.row_stride * item,)
    else:
        strides = (t.row_stride * item, t.col_stride * item)
    return np.lib.stride_tricks.as_strided(flat, shape=t.shape, strides=strides, writeable=False)


def _as_2d(a: np.ndarray) -> np.ndarray:
    return a.reshape(a.shape[0], 1) if a.ndim == 1 else a


def _operand(storage: dict, o, mode: str, primary_shape):
    """Value of a secondary operand broadcast against the primary."""
    if not hasattr(o, "buffer_key"):  # Scalar
        return F32(o.value)
    v = _view(storage[o.buffer_key], o)
    if mode == "none":
        return v
    return np.broadcast_to(_as_2d(v) if mode == "col" else v, primary_shape)


def evaluate(ops, inputs: dict | None = None) -> dict:
    """Evaluate every op of ``ops`` (an ``Operations``) on the CPU.

    ``inputs`` maps storage-owner names to arrays (default: ``ops.uploads``).
    Returns ``{tensor name: ndarray}`` for every produced tensor and every
    view of a produced tensor.  Matmul results are float64; everything else
    float32."""
    from metellus_amd.orchestrator.ir import ElementwiseOp, MatmulOp, ReductionOp, ShapeOp

    storage: dict[str, np.ndarray] = {}
    src = ops.uploads if inputs is None else inputs
    for name, arr in src.items():
        storage[name] = np.ascontiguousarray(arr, dtype=F32)
    out: dict[str, np.ndarray] = {}
    for op in ops.build():
        if isinstance(op, MatmulOp):
            a = _view(storage[op.a.buffer_key], op.a).astype(np.float64)
            b = _view(storage[op.b.buffer_key], op.b).astype(np.float64)
            res = a @ b
            storage[op.out.buffer_key] = res.astype(F32)
            out[op.out.name] = res
            continue
        if isinstance(op, ElementwiseOp):
            x = _view(storage[op.operands[0].buffer_key], op.operands[0])
            y = cond = None
            if len(op.operands) >= 2:
                y = _operand(storage, op.operands[1], op.y_broadcast.value, x.shape)
            if len(op.operands) == 3:
                cond = _operand(storage, op.operands[2], op.cond_broadcast.value, x.shape)
            res = apply_elementwise(op.op, x, y, cond)
        elif isinstance(op, ReductionOp):
            x = _view(storage[op.input.buffer_key], op.input)
            res = reduce_rows(x, op.op)
        elif isinstance(op, ShapeOp):
            x = _view(storage[op.input.buffer_key], op.input)
            res = np.ascontiguousarray(x).reshape(op.out.shape)
        else:
            raise TypeError(f"unknown op {op!r}")
        storage[op.out.buffer_key] = np.ascontiguousarray(res, dtype=F32).reshape(op.out.shape)
        out[op.out.name] = res
    for name, t in ops.tensors.items():
        if name not in out and t.buffer_key in storage and t.buffer_key != name and t.buffer_key not in src:
            out[name] = np.ascontiguousarray(_view(storage[t.buffer_key], t))
    return out


# ---------------------------------------------------------------------------
# tolerances
# ---------------------------------------------------------------------------


def matmul_tolerance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Per-element bound 1e-4 * sqrt(K) * (|A| @ |B|): the stated fp32 matmul
    tolerance applied to the magnitude the sum is built from."""
    K = a.shape[1]
    return 1e-4 * np.sqrt(K) * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
