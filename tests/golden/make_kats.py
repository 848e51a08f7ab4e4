"""Generate tests/golden/kats.npz: known-answer cases for the elementwise and
reduction semantics.

Inputs are built exactly as the reference's edge-case probes build them
(reference: sandbox.py, probe functions named per case below); expected
outputs are closed forms fixed by IEEE-754 float32 arithmetic and the
reference op table (reference: src/compute/elementwise/elementwise.py:18-58),
computed here directly -- NOT with oracle/ir_eval.py, which these fixtures
check.

Run:  python tests/golden/make_kats.py   (rewrites kats.npz)
"""

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F = np.float32
INF, NAN = F(np.inf), F(np.nan)


def cases():
    out = {}

    # p21_tanh_extreme_values: saturates at +/-1 (no NaN), tanh(0) = 0
    X = np.zeros((16, 32), dtype=F)
    X[0, :16] = np.array(
        [0.0, 1.0, -1.0, 10.0, -10.0, 60.0, -60.0, 80.0, -80.0, 100.0, -100.0, 200.0, 1e-10, -1e-10, 0.5, -0.5],
        dtype=F,
    )
    X[1, :] = np.linspace(-100.0, 100.0, 32, dtype=F)
    out["tanh_extremes"] = dict(op="tanh", x=X, expected=np.tanh(X.astype(np.float64)).astype(F), atol=1e-6)

    # p108_div_by_zero_handling: IEEE division (divisors are 0.5 or 1 here)
    X = np.array(
        [
            [1.0, -1.0, 2.0, 0.0, -2.0, 3.0, -3.0, 4.0],
            [-4.0, 5.0, -5.0, 6.0, -6.0, 7.0, -7.0, 8.0],
            [-8.0, 9.0, -9.0, 10.0, -10.0, 11.0, -11.0, 12.0],
            [1e30, -1e30, 1e-30, -1e-30, 0.0, 0.0, 0.0, 0.0],
        ],
        dtype=F,
    )
    Z = np.zeros((4, 8), dtype=F)
    Z[0, 3] = 1.0
    Z[3, 4] = 1.0
    Y = np.where(Z == 0, F(0.5), Z).astype(F)
    # x / 0.5 == 2x exactly; x / 1 == x
    out["div_half_or_one"] = dict(op="div", x=X, y=Y, expected=np.where(Y == 1, X, X * F(2)).astype(F), atol=0.0)

    # true division by zero: +-inf, and 0/0 = NaN
    X = np.array([[1.0, -1.0, 0.0, 2.0]], dtype=F)
    Y = np.zeros((1, 4), dtype=F)
    out["div_by_zero"] = dict(op="div", x=X, y=Y, expected=np.array([[INF, -INF, NAN, INF]], dtype=F), atol=0.0)

    rng = np.random.default_rng(42)
    X = rng.standard_normal((16, 16)).astype(F)
    out["min_with_inf"] = dict(op="min", x=X, scalar=float("inf"), expected=X.copy(), atol=0.0)  # p251
    out["max_with_neg_inf"] = dict(op="max", x=X, scalar=float("-inf"), expected=X.copy(), atol=0.0)  # p252

    N8 = np.full((8, 8), NAN, dtype=F)
    out["equal_nan"] = dict(op="equal", x=N8, scalar=float("nan"), expected=np.zeros((8, 8), F), atol=0.0)  # p255
    out["not_equal_nan"] = dict(op="not_equal", x=N8, scalar=float("nan"), expected=np.ones((8, 8), F), atol=0.0)  # p256
    out["zero_times_inf"] = dict(  # p257
        op="mul", x=np.zeros((8, 8), F), y=np.full((8, 8), INF, F), expected=np.full((8, 8), NAN, F), atol=0.0
    )
    out["recip_inf"] = dict(op="recip", x=np.full((8, 8), INF, F), expected=np.zeros((8, 8), F), atol=0.0)  # p259
    out["log_zero"] = dict(op="log", x=np.zeros((8, 8), F), expected=np.full((8, 8), -INF, F), atol=0.0)  # p260

    # p266_where_operand_is_nan_tensor: where(x, y, cond) = cond != 0 ? x : y
    cond = np.array([[1.0, 0.0, 1.0, 0.0]] * 4, dtype=F)
    x = np.full((4, 4), NAN, F)
    y = np.ones((4, 4), F)
    out["where_nan"] = dict(op="where", x=x, y=y, cond=cond, expected=np.array([[NAN, 1, NAN, 1]] * 4, F), atol=0.0)

    # reference op table: fmax/fmin drop NaN; sign(NaN) = 0
    x = np.array([[NAN, 1.0, -2.0, NAN]], F)
    y = np.array([[1.0, NAN, NAN, NAN]], F)
    out["fmax_nan"] = dict(op="max", x=x, y=y, expected=np.array([[1.0, 1.0, -2.0, NAN]], F), atol=0.0)
    out["fmin_nan"] = dict(op="min", x=x, y=y, expected=np.array([[1.0, 1.0, -2.0, NAN]], F), atol=0.0)
    x = np.array([[NAN, -0.0, 0.0, -3.5, 2.0, INF, -INF, 1e-40]], F)
    out["sign_cases"] = dict(op="sign", x=x, expected=np.array([[0, 0, 0, -1, 1, 1, -1, 1]], F), atol=0.0)

    # p265_reduce_sum_with_nan_input
    X = np.array([[NAN, 1.0, 2.0, 3.0], [4.0, 5.0, 6.0, 7.0]], dtype=F)
    out["sum_with_nan"] = dict(op="reduce_sum", x=X, expected=np.array([NAN, 22.0], F), atol=0.0)
    # integer-valued data: every partial sum exact in float32, so any order gives the exact sum
    X = np.arange(2 * 300, dtype=F).reshape(2, 300) % 17 - 8
    out["sum_exact_integers"] = dict(
        op="reduce_sum", x=X, expected=np.array([float(sum(r)) for r in X.astype(np.int64)], F), atol=0.0
    )
    P = np.array([[2.0] * 10 + [0.5] * 10], F)
    out["product_powers_of_two"] = dict(op="reduce_product", x=P, expected=np.array([1.0], F), atol=0.0)
    return out


def main():
    flat = {}
    for name, case in cases().items():
        for key, val in case.items():
            flat[f"{name}/{key}"] = np.asarray(val)
    np.savez(os.path.join(HERE, "kats.npz"), **flat)
    print(f"wrote {len(cases())} cases")


if __name__ == "__main__":
    main()
