"""Whole-output checks of fp32 matmul results (test infrastructure).

Every element of a GPU product ``C ~ (A @ B) * scale`` is compared with the
float64 product of the same float32 operands, against two bounds:

* the stated matmul bar, ``1e-4 * sqrt(K) * (|A| @ |B|)``;
* the float32 accumulation bound, ``2 * gamma_K * (|A| @ |B|)`` with
  ``gamma_K = K u / (1 - K u)``, u = 2^-24 (Higham, *Accuracy and Stability
  of Numerical Algorithms*, 2nd ed., eq. 3.5): a K-term dot product summed
  in float32 in *any* order -- MFMA blocks, k-chunks, stream-K partial tiles
  added in any grouping -- is within ``gamma_K * sum |a_k b_k|`` of the exact
  value when every product and every addition rounds with relative error at
  most u; the factor 2 allows each to round with up to 2u.

The second bound is tighter than the first by about 26x at K = 4096, so a
missing or duplicated 32-wide k-chunk contribution (an error of the size of
a 32-term partial sum) fails it on almost every element of the affected
tile, where the stated bar alone lets most of them through.  A check of the
whole output instead of sampled rows means no tile is left unchecked.

Why not Freivalds (``C r`` against ``A (B r)``): for random data the
deterministic bound on ``|E r|`` sums the per-element bounds over all N
columns, while a corrupted 256-column tile moves ``C r`` by only about
sqrt(256) times its per-element error -- a zeroed tile of a 4096^3 product
of N(0, 1) operands (``C r`` moves by ~1e3) hides under a bound of ~5e4.
The full float64 product costs O(MNK) on the host (well under a minute for
the benchmark configurations) and settles every element.
"""

from __future__ import annotations

import numpy as np

U32 = 2.0**-24  # unit roundoff of float32


def accumulation_bound(K: int) -> float:
    """2 * gamma_K for a K-term float32 dot product."""
    ku = K * U32
    assert ku < 0.5, "gamma_K is defined for K u < 1"
    return 2.0 * ku / (1.0 - ku)


def check_matmul(
    got: np.ndarray,
    a: np.ndarray,
    b: np.ndarray,
    what: str,
    *,
    scale: float = 1.0,
    a_rel: float = 0.0,
    block: int = 1024,
) -> None:
    """Assert both bounds for every element of ``got`` (M x N, float32).

    ``scale``: the product was multiplied by this float32 constant in the
    epilogue (one more rounding: u |C|).  ``a_rel``: the kernel's A operand
    may differ from ``a`` by this relative amount per element (a prologue
    computed with a bounded-error operation), which adds
    ``a_rel * (|A| @ |B|)``."""
    M, K = a.shape
    assert b.shape[0] == K and got.shape == (M, b.shape[1]), (got.shape, a.shape, b.shape)
    b64 = b.astype(np.float64)
    babs = np.abs(b64)
    stated_k = 1e-4 * np.sqrt(K)
    tight_k = accumulation_bound(K) + a_rel
    s = float(scale)
    for r0 in range(0, M, block):
        a64 = a[r0 : r0 + block].astype(np.float64)
        ref = (a64 @ b64) * s
        mag = (np.abs(a64) @ babs) * abs(s)
        err = np.abs(got[r0 : r0 + block].astype(np.float64) - ref)
        rounding = np.abs(ref) * (2 * U32 if s != 1.0 else 0.0) + 1e-30
        over = err > stated_k * mag + rounding
        assert not over.any(), (
            f"{what}: {int(over.sum())} elements over the stated matmul bar in rows {r0}..; "
            f"max err {err.max():.3e}; first (row, col, got, ref): {_first_bad(over, got, ref, r0)}"
        )
        over = err > tight_k * mag + rounding
        assert not over.any(), (
            f"{what}: {int(over.sum())} elements over the float32 accumulation bound in rows {r0}..; "
            f"first at {np.argwhere(over)[0] + [r0, 0]}, max err {err.max():.3e}"
        )


def _first_bad(over: np.ndarray, got: np.ndarray, ref: np.ndarray, r0: int, n: int = 12) -> list:
    """The first ``n`` (row, col, got, ref) where ``over`` holds, rows
    counted from the block at ``r0``."""
    return [(int(r) + r0, int(c), float(got[r0 + r, c]), round(float(ref[r, c]), 6))
            for r, c in np.argwhere(over)[:n]]


def check_matmul_product(
    got: np.ndarray, x: np.ndarray, w1: np.ndarray, w2: np.ndarray, what: str, *, block: int = 1024
) -> None:
    """Assert ``got ~ (x @ w1) * (x @ w2)`` (the diamond: two fp32 products
    multiplied in the epilogue) for every element: with per-product bounds
    t1, t2, |err| <= |h2| t1 + |h1| t2 + t1 t2 + 2u |h1 h2|, for t the stated
    bar and, separately, the accumulation bound."""
    M, K = x.shape
    w1_64, w2_64 = w1.astype(np.float64), w2.astype(np.float64)
    a1, a2 = np.abs(w1_64), np.abs(w2_64)
    for r0 in range(0, M, block):
        x64 = x[r0 : r0 + block].astype(np.float64)
        h1, h2 = x64 @ w1_64, x64 @ w2_64
        xa = np.abs(x64)
        m1, m2 = xa @ a1, xa @ a2
        err = np.abs(got[r0 : r0 + block].astype(np.float64) - h1 * h2)
        for coef, name in ((1e-4 * np.sqrt(K), "stated matmul bar"), (accumulation_bound(K), "accumulation bound")):
            t1, t2 = coef * m1, coef * m2
            bound = np.abs(h2) * t1 + np.abs(h1) * t2 + t1 * t2 + np.abs(h1 * h2) * 2 * U32 + 1e-30
            over = err > bound
            assert not over.any(), (
                f"{what}: {int(over.sum())} elements over the {name} in rows {r0}..; max err {err.max():.3e}"
            )
