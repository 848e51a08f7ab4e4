"""Edge-case programs restated from the reference's correctness sweep
(reference: sandbox.py, probes p01..p266; each probe there builds an
``Operations`` program and compares chosen outputs with MLX at
rtol = atol = 1e-3, NaN equal to NaN -- sandbox.py:40-49).

Here each probe is a function over a ``Probe`` builder; the expected values
come from the CPU oracle (``oracle/ir_eval.evaluate``) on the same inputs.
Probe names keep the reference's numbers so each can be traced to
sandbox.py.  Inputs are drawn from ``default_rng(0)`` as in the reference,
with the hand-picked edge values where the probe depends on them.
"""

from __future__ import annotations

from typing import Callable

import numpy as np

from metellus_amd.orchestrator import Operations

F32 = np.float32


class Probe:
    def __init__(self, seed: int = 0) -> None:
        self.ops = Operations()
        self.rng = np.random.default_rng(seed)
        self.checks: list[str] = []
        self.exact: set[str] = set()

    def reseed(self, seed: int) -> None:
        """Probes p200 and later draw some inputs from ``default_rng(42)``."""
        self.rng = np.random.default_rng(seed)

    # ---- inputs
    def arr(self, name: str, a) -> np.ndarray:
        a = np.ascontiguousarray(np.asarray(a, dtype=F32))
        self.ops.from_numpy(a, name)
        return a

    def randn(self, name: str, *shape: int) -> np.ndarray:
        return self.arr(name, self.rng.standard_normal(shape))

    def uniform(self, name: str, lo: float, hi: float, *shape: int) -> np.ndarray:
        return self.arr(name, self.rng.uniform(lo, hi, shape))

    # ---- ops
    def mm(self, a: str, b: str, out: str) -> None:
        self.ops.matmul(a=a, b=b, out=out)

    def ew(self, op: str, out: str, *operands, y: str | None = None, cond: str | None = None) -> None:
        kw = {}
        if y is not None:
            kw["y_broadcast"] = y
        if cond is not None:
            kw["cond_broadcast"] = cond
        self.ops.elementwise(op, out=out, operands=tuple(operands), **kw)

    def red(self, op: str, out: str, x: str) -> None:
        self.ops.reduction(op, out=out, x=x, axis=-1)

    def t(self, x: str, out: str) -> None:
        self.ops.transpose(x, out=out)

    def rs(self, x: str, shape: tuple[int, ...], out: str) -> None:
        self.ops.reshape(x, shape, out=out)

    # ---- what the probe verifies
    def check(self, *names: str, exact: bool = False) -> None:
        self.checks.extend(names)
        if exact:
            self.exact.update(names)


PROBES: dict[str, Callable[[Probe], None]] = {}


def probe(fn: Callable[[Probe], None]) -> Callable[[Probe], None]:
    PROBES[fn.__name__] = fn
    return fn


def build(name: str) -> Probe:
    p = Probe()
    PROBES[name](p)
    return p


# ---------------------------------------------------------------------------
# p01 .. p84
# ---------------------------------------------------------------------------


@probe
def p01_product_reduction(p):
    p.uniform("X", 0.7, 1.3, 16, 8)
    p.red("product", "prod", "X")
    p.check("prod")


@probe
def p02_where_ternary(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.arr("Cond", p.rng.standard_normal((16, 32)) > 0)
    p.ew("where", "out", "X", "Y", "Cond")
    p.check("out", exact=True)


@probe
def p03_comparison_mask(p):
    p.randn("X", 16, 32)
    p.ew("lt", "mask", "X", 0.5)
    p.ew("mul", "masked", "X", "mask")
    p.check("mask", "masked", exact=True)


@probe
def p04_reduction_on_transposed(p):
    p.randn("X", 32, 48)
    p.t("X", "Xt")
    p.red("sum", "col_sums", "Xt")
    p.check("col_sums")


@probe
def p05_row_broadcast_via_reshape(p):
    M, N = 32, 64
    p.randn("X", N, M)
    p.red("sum", "col_sum_1d", "X")
    p.rs("col_sum_1d", (1, N), "col_sum_row")
    p.randn("Z", M, N)
    p.ew("add", "adjusted", "Z", "col_sum_row", y="row")
    p.check("adjusted")


def _two_matmuls(p, shared: bool, merge: str, n: int = 64):
    if shared:
        p.randn("A", n, n)
        p.randn("B1", n, n)
        p.randn("B2", n, n)
        p.mm("A", "B1", "t1")
        p.mm("A", "B2", "t2")
    else:
        p.randn("A1", n, n)
        p.randn("B1", n, n)
        p.randn("A2", n, n)
        p.randn("B2", n, n)
        p.mm("A1", "B1", "t1")
        p.mm("A2", "B2", "t2")
    p.ew(merge, "out", "t1", "t2")
    p.check("out")


@probe
def p06_diamond_shared_a(p):
    _two_matmuls(p, True, "add")


@probe
def p07_multi_producer_no_shared(p):
    _two_matmuls(p, False, "mul")


@probe
def p08_one_row_matrix(p):
    p.randn("X", 1, 64)
    p.randn("Y", 1, 64)
    p.ew("add", "z", "X", "Y")
    p.check("z", exact=True)


@probe
def p09_one_col_matrix(p):
    p.randn("X", 64, 1)
    p.randn("Y", 64, 1)
    p.ew("add", "z", "X", "Y")
    p.check("z", exact=True)


@probe
def p10_full_tensor_mean_broadcast(p):
    M = 16
    p.randn("X", M, 32)
    p.red("sum", "row_sum_1d", "X")
    p.rs("row_sum_1d", (1, M), "row_sum_row")
    p.check("row_sum_1d")


@probe
def p11_relu_then_reduce(p):
    p.randn("X", 32, 48)
    p.ew("max", "relu_X", "X", 0.0)
    p.red("sum", "s", "relu_X")
    p.check("s")


@probe
def p12_reduce_then_scaled(p):
    p.randn("X", 32, 64)
    p.red("sum", "s", "X")
    p.ew("mul", "mean", "s", 1.0 / 64)
    p.check("mean")


@probe
def p13_chain_with_intermediate_reuse(p):
    p.randn("X", 32, 64)
    p.randn("bias", 1, 64)
    p.ew("add", "t", "X", "bias", y="row")
    p.ew("mul", "y", "t", "X")
    p.check("y", exact=True)


@probe
def p14_matmul_then_transpose_then_add(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.randn("D", 64, 64)
    p.mm("A", "B", "C")
    p.t("C", "Ct")
    p.ew("add", "out", "D", "Ct")
    p.check("out")


@probe
def p15_reshape_op_via_transpose_then_reshape(p):
    M, N = 16, 24
    p.randn("X", M, N)
    p.t("X", "Xt")
    p.rs("Xt", (N * M,), "flat")
    p.check("flat", exact=True)


@probe
def p16_recompute_lane_agnostic_prologue(p):
    p.randn("X", 64, 64)
    p.randn("B1", 64, 64)
    p.randn("B2", 64, 64)
    p.ew("max", "X1", "X", 0.0)
    p.mm("X1", "B1", "t1")
    p.mm("X1", "B2", "t2")
    p.check("t1", "t2")


@probe
def p17_softmax_via_primitives(p):
    M = 32
    p.randn("X", M, 64)
    p.red("max", "row_max_1d", "X")
    p.rs("row_max_1d", (M, 1), "row_max")
    p.ew("subtract", "shifted", "X", "row_max", y="col")
    p.ew("exp", "e", "shifted")
    p.red("sum", "row_sum_1d", "e")
    p.rs("row_sum_1d", (M, 1), "row_sum")
    p.ew("div", "probs", "e", "row_sum", y="col")
    p.check("probs")


@probe
def p18_double_transpose_identity(p):
    p.randn("X", 16, 24)
    p.t("X", "Xt")
    p.t("Xt", "Xtt")
    p.ew("add", "out", "Xtt", "Xtt")
    p.check("out", exact=True)


@probe
def p19_min_reduction(p):
    p.randn("X", 32, 48)
    p.red("min", "rowmins", "X")
    p.check("rowmins", exact=True)


@probe
def p20_unary_negate_chain(p):
    p.randn("X", 16, 32)
    p.ew("negate", "nx", "X")
    p.ew("negate", "nnx", "nx")
    p.check("nnx", exact=True)


@probe
def p21_tanh_extreme_values(p):
    x = np.zeros((16, 32), F32)
    x[0, :16] = [0.0, 1.0, -1.0, 10.0, -10.0, 60.0, -60.0, 80.0, -80.0, 100.0, -100.0, 200.0,
                 1e-10, -1e-10, 0.5, -0.5]
    x[1, :] = np.linspace(-100.0, 100.0, 32, dtype=F32)
    p.arr("X", x)
    p.ew("tanh", "th", "X")
    p.check("th")


@probe
def p22_reduce_epilogue_chain(p):
    p.randn("X", 32, 64)
    p.red("sum", "s", "X")
    p.ew("mul", "s2", "s", 2.0)
    p.ew("add", "s3", "s2", 1.0)
    p.check("s3")


@probe
def p23_prologue_chain_into_matmul(p):
    p.randn("X", 64, 64)
    p.randn("B", 64, 64)
    p.ew("mul", "X1", "X", 2.0)
    p.ew("add", "X2", "X1", 1.0)
    p.mm("X2", "B", "C")
    p.check("C")


@probe
def p24_mixed_epilogue_chain(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.randn("bias", 1, 64)
    p.mm("A", "B", "z")
    p.ew("add", "zb", "z", "bias", y="row")
    p.ew("max", "y", "zb", 0.0)
    p.check("y")


@probe
def p25_sum_of_comparison(p):
    p.randn("X", 32, 64)
    p.ew("gt", "mask", "X", 0.0)
    p.red("sum", "count", "mask")
    p.check("count", exact=True)


@probe
def p26_reshape_col_to_1d(p):
    p.randn("X", 32, 1)
    p.randn("Y", 32)
    p.rs("X", (32,), "X1d")
    p.ew("add", "z", "X1d", "Y")
    p.check("z", exact=True)


@probe
def p27_reshape_to_same_shape(p):
    p.randn("X", 16, 32)
    p.rs("X", (16, 32), "X_alias")
    p.ew("mul", "y", "X_alias", 3.0)
    p.check("y", exact=True)


@probe
def p28_non_aligned_matmul_with_epilogue_chain(p):
    p.randn("A", 33, 49)
    p.randn("B", 49, 41)
    p.mm("A", "B", "z")
    p.ew("max", "z_r", "z", 0.0)
    p.ew("add", "z_a", "z_r", 0.5)
    p.ew("mul", "y", "z_a", 0.25)
    p.check("y")


@probe
def p29_matmul_with_transposed_input_b(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.t("B", "Bt")
    p.mm("A", "Bt", "C")
    p.check("C")


@probe
def p30_where_with_broadcast_cond(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.arr("cond", p.rng.standard_normal((1, 32)) > 0)
    p.ew("where", "out", "X", "Y", "cond", cond="row")
    p.check("out", exact=True)


@probe
def p31_matmul_input_used_twice_as_a_and_b(p):
    p.randn("X", 64, 64)
    p.mm("X", "X", "C")
    p.check("C")


@probe
def p32_self_add(p):
    p.randn("X", 16, 32)
    p.ew("add", "y", "X", "X")
    p.check("y", exact=True)


@probe
def p33_recompute_two_consumers_one_unfusable(p):
    p.randn("X", 64, 64)
    p.randn("B", 64, 64)
    p.randn("C", 64, 64)
    p.ew("max", "X1", "X", 0.0)
    p.mm("X1", "B", "t1")
    p.ew("add", "t2", "X1", "C")
    p.check("t1", "t2")


@probe
def p34_subtract_scalar_first(p):
    p.arr("X", p.rng.standard_normal((16, 32)).astype(F32) + F32(100.0))
    p.ew("subtract", "y", "X", 5.0)
    p.check("y", exact=True)


@probe
def p36_gram_matrix_x_xt(p):
    p.randn("X", 64, 32)
    p.t("X", "Xt")
    p.mm("X", "Xt", "C")
    p.check("C")


@probe
def p37_matmul_M_eq_1(p):
    p.randn("A", 1, 64)
    p.randn("B", 64, 64)
    p.mm("A", "B", "C")
    p.check("C")


@probe
def p38_matmul_N_eq_1(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 1)
    p.mm("A", "B", "C")
    p.check("C")


@probe
def p39_reduce_over_k_eq_1(p):
    p.randn("X", 64, 1)
    p.red("sum", "s", "X")
    p.check("s", exact=True)


@probe
def p40_two_relus_share_input(p):
    p.randn("X", 16, 32)
    p.ew("max", "r1", "X", 0.0)
    p.ew("max", "r2", "X", 0.5)
    p.check("r1", "r2", exact=True)


@probe
def p41_chain_with_4_ops(p):
    p.randn("X", 16, 32)
    p.ew("add", "a", "X", 1.0)
    p.ew("mul", "b", "a", 2.0)
    p.ew("max", "c", "b", 0.0)
    p.ew("exp", "y", "c")
    p.check("y")


@probe
def p42_reduction_then_two_view_consumers(p):
    M = 16
    p.randn("X", M, 32)
    p.randn("Y", M, M)
    p.randn("Z", M, M)
    p.red("sum", "rs", "X")
    p.rs("rs", (M, 1), "rs_col")
    p.rs("rs", (1, M), "rs_row")
    p.ew("add", "A", "Y", "rs_col", y="col")
    p.ew("add", "B", "Z", "rs_row", y="row")
    p.check("A", "B")


@probe
def p43_pow_op(p):
    p.arr("X", np.abs(p.rng.standard_normal((16, 32))).astype(F32) + F32(0.1))
    p.ew("pow", "y", "X", 0.5)
    p.check("y")


@probe
def p44_sign_of_zero(p):
    p.arr("X", [[-2.0, -1.0, -0.5, -0.0, 0.0, 0.5, 1.0, 2.0],
                [-3.0, -1e-30, 1e-30, 0.0, -0.0, 1.0, -1.0, 100.0],
                [-1e10, 1e10, 0.0, 0.0, 0.0, 0.0, -0.0, -0.0],
                [1.0, 2.0, 3.0, 4.0, -1.0, -2.0, -3.0, -4.0]])
    p.ew("sign", "y", "X")
    p.check("y", exact=True)


@probe
def p45_chain_uses_scalar_operand_with_negate(p):
    p.randn("X", 16, 32)
    p.ew("subtract", "t", "X", 5.0)
    p.ew("negate", "y", "t")
    p.check("y", exact=True)


@probe
def p46_recip_op(p):
    p.uniform("X", 0.5, 2.0, 16, 32)
    p.ew("recip", "y", "X")
    p.check("y", exact=True)


@probe
def p47_sqrt_chain_log(p):
    p.uniform("X", 0.1, 10.0, 16, 32)
    p.ew("sqrt", "r", "X")
    p.ew("log", "y", "r")
    p.check("y")


@probe
def p49_diamond_shared_a_small(p):
    _two_matmuls(p, True, "add", n=16)


@probe
def p50_multi_producer_small(p):
    _two_matmuls(p, False, "add", n=16)


@probe
def p51_prologue_same_input_into_both_a_and_b(p):
    p.randn("X", 32, 32)
    p.ew("add", "X1", "X", 1.0)
    p.mm("X1", "X1", "C")
    p.check("C")


@probe
def p52_elementwise_extra_shares_input_buffer(p):
    p.randn("X", 16, 32)
    p.rs("X", (16, 32), "X_alias")
    p.ew("add", "y", "X", "X_alias")
    p.check("y", exact=True)


@probe
def p53_matmul_with_bias_that_also_is_input_a(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "z")
    p.ew("add", "y", "z", "A", y="none")
    p.check("y")


@probe
def p54_equal_op(p):
    p.arr("X", np.tile(np.arange(16, dtype=F32), (8, 1)))
    p.ew("equal", "mask", "X", 4.0)
    p.check("mask", exact=True)


@probe
def p55_chain_then_chain_via_reduction(p):
    p.randn("X", 32, 64)
    p.ew("max", "r", "X", 0.0)
    p.ew("mul", "r2", "r", 2.0)
    p.red("sum", "s", "r2")
    p.ew("mul", "y", "s", 0.5)
    p.check("y")


@probe
def p60_reduction_prologue_full_shape_extra(p):
    p.randn("X", 32, 64)
    p.randn("Y", 32, 64)
    p.ew("add", "XY", "X", "Y")
    p.red("sum", "s", "XY")
    p.check("s")


@probe
def p62_multi_anchor_same_b(p):
    p.randn("A1", 16, 16)
    p.randn("A2", 16, 16)
    p.randn("B", 16, 16)
    p.mm("A1", "B", "t1")
    p.mm("A2", "B", "t2")
    p.ew("add", "out", "t1", "t2")
    p.check("out")


@probe
def p63_comparison_into_max(p):
    p.randn("X", 16, 32)
    p.ew("gt", "mask", "X", 0.0)
    p.ew("max", "y", "X", "mask")
    p.check("y", exact=True)


@probe
def p64_chain_through_view(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("add", "t1", "X", "Y")
    p.rs("t1", (16, 32), "t2")
    p.ew("mul", "t3", "t2", 2.0)
    p.check("t3", exact=True)


@probe
def p65_chain_with_first_op_as_comparison(p):
    p.randn("X", 16, 32)
    p.ew("gt", "mask", "X", 0.0)
    p.ew("add", "y", "mask", 5.0)
    p.check("y", exact=True)


@probe
def p66_input_used_as_col_broadcast_into_matmul_epilogue(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.randn("bias", 64, 1)
    p.mm("A", "B", "z")
    p.ew("add", "y", "z", "bias", y="col")
    p.check("y")


@probe
def p67_input_used_as_scalar_broadcast(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.arr("s", [[1.5]])
    p.mm("A", "B", "z")
    p.ew("add", "y", "z", "s", y="scalar")
    p.check("y")


@probe
def p68_elementwise_chain_with_col_broadcast_intermediate_use(p):
    p.randn("X", 16, 32)
    p.randn("b", 16, 1)
    p.ew("add", "t1", "X", "b", y="col")
    p.ew("add", "t2", "t1", "b", y="col")
    p.check("t2", exact=True)


@probe
def p69_reduce_max_all_negatives(p):
    p.arr("X", -np.abs(p.rng.standard_normal((16, 64)).astype(F32)) - F32(0.1))
    p.red("max", "rm", "X")
    p.check("rm", exact=True)


@probe
def p70_reduction_with_K_less_than_simdwidth(p):
    p.randn("X", 16, 7)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p71_reduction_K_between_32_and_128(p):
    p.randn("X", 16, 50)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p72_matmul_tg_epilogue_reads_input_a_again(p):
    a = p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.arr("bias", a[0:1, :])
    p.mm("A", "B", "z")
    p.ew("add", "y", "z", "bias", y="row")
    p.check("y")


@probe
def p73_input_buffer_size_only_uses_first_K_elements(p):
    p.randn("X", 16, 32)
    p.ew("add", "y", "X", 0.0)
    p.check("y", exact=True)


@probe
def p75_multi_anchor_a0_eq_b1(p):
    p.randn("X", 16, 16)
    p.randn("Y", 16, 16)
    p.randn("Z", 16, 16)
    p.t("X", "Xt")
    p.mm("X", "Y", "t1")
    p.mm("Z", "Xt", "t2")
    p.ew("add", "out", "t1", "t2")
    p.check("out")


@probe
def p76_chain_with_tail_consumed_by_view_then_op(p):
    p.randn("X", 16, 32)
    p.ew("add", "t1", "X", 1.0)
    p.rs("t1", (16, 32), "t2")
    p.ew("mul", "t3", "t2", 2.0)
    p.check("t3", exact=True)


@probe
def p77_relu_then_reshape_then_relu(p):
    p.randn("X", 8, 16)
    p.ew("max", "t1", "X", 0.0)
    p.rs("t1", (128,), "t1_flat")
    p.ew("max", "t2", "t1_flat", 0.0)
    p.check("t2", exact=True)


@probe
def p78_reduce_then_use_result_in_two_chains(p):
    p.randn("X", 16, 32)
    p.red("sum", "rs", "X")
    p.ew("mul", "y1", "rs", 2.0)
    p.ew("add", "y2", "rs", 1.0)
    p.check("y1", "y2")


@probe
def p79_matmul_with_row_broadcast_full_M_eq_N(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.randn("bias", 1, 32)
    p.mm("A", "B", "z")
    p.ew("add", "y", "z", "bias", y="row")
    p.check("y")


@probe
def p80_chained_reductions_on_diff_axes(p):
    p.randn("X", 8, 16)
    p.red("sum", "rs", "X")
    p.rs("rs", (1, 8), "rs_row")
    p.red("sum", "total", "rs_row")
    p.check("total")


@probe
def p81_transpose_of_1d_reshape_view(p):
    p.randn("X", 16)
    p.randn("Y", 4, 4)
    p.rs("X", (4, 4), "X2d")
    p.t("X2d", "X2dT")
    p.ew("add", "z", "Y", "X2dT")
    p.check("z", exact=True)


@probe
def p82_reduce_then_negate_epilogue(p):
    p.randn("X", 16, 32)
    p.red("sum", "rs", "X")
    p.ew("negate", "y", "rs")
    p.check("y")


@probe
def p83_chain_writes_back_to_same_position(p):
    p.randn("X", 16, 32)
    p.ew("max", "y", "X", 0.0)
    p.ew("exp", "z", "X")
    p.check("y", exact=True)
    p.check("z")


@probe
def p84_not_equal_op(p):
    p.arr("X", p.rng.choice([-1.0, 0.0, 1.0, 2.0], size=(16, 32)))
    p.ew("not_equal", "mask", "X", 0.0)
    p.check("mask", exact=True)


# ---------------------------------------------------------------------------
# p35 .. p99 (the reference defines these out of numeric order)
# ---------------------------------------------------------------------------


@probe
def p35_div_by_tensor(p):
    p.randn("X", 16, 32)
    p.uniform("Y", 0.5, 2.0, 16, 32)
    p.ew("div", "z", "X", "Y")
    p.check("z", exact=True)


@probe
def p48_reduce_then_reshape_then_reduce(p):
    p.randn("X", 16, 32)
    p.red("sum", "rs", "X")
    p.rs("rs", (1, 16), "rs_row")
    p.red("sum", "total", "rs_row")
    p.check("total")


def _prologue_matmul(p, extra_shape, y_mode, side="a"):
    p.randn("X", 32, 32)
    p.randn("E", *extra_shape)
    p.randn("B", 32, 32)
    if side == "a":
        p.ew("add", "Xe", "X", "E", y=y_mode)
        p.mm("Xe", "B", "C")
    else:
        p.ew("mul", "Be", "B", "E", y=y_mode)
        p.mm("X", "Be", "C")
    p.check("C")


@probe
def p56_matmul_prologue_with_full_shape_extra(p):
    _prologue_matmul(p, (32, 32), "none")


@probe
def p57_matmul_prologue_row_broadcast_extra(p):
    _prologue_matmul(p, (1, 32), "row")


@probe
def p58_matmul_prologue_col_broadcast_extra(p):
    _prologue_matmul(p, (32, 1), "col")


@probe
def p59_matmul_prologue_b_side_row_broadcast(p):
    _prologue_matmul(p, (1, 32), "row", side="b")


@probe
def p61_matmul_prologue_chain_with_tensor_then_scalar(p):
    p.randn("X", 32, 32)
    p.randn("Y", 32, 32)
    p.randn("B", 32, 32)
    p.ew("add", "X1", "X", "Y")
    p.ew("mul", "X2", "X1", 2.0)
    p.mm("X2", "B", "C")
    p.check("C")


@probe
def p74_reshape_2d_to_2d_view(p):
    p.randn("X", 4, 8)
    p.rs("X", (32, 1), "X_col")
    p.randn("Y", 32, 8)
    p.ew("add", "z", "Y", "X_col", y="col")
    p.check("z", exact=True)


@probe
def p85_matmul_K_eq_tileK(p):
    p.randn("A", 32, 16)
    p.randn("B", 16, 32)
    p.mm("A", "B", "C")
    p.check("C")


@probe
def p86_elementwise_transpose_as_primary(p):
    p.randn("X", 16, 32)
    p.randn("Y", 32, 16)
    p.t("X", "Xt")
    p.ew("add", "z", "Xt", "Y")
    p.check("z", exact=True)


@probe
def p87_reduction_M_eq_1(p):
    p.randn("X", 1, 64)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p88_matmul_1x1_at_1x1(p):
    p.arr("A", [[2.0]])
    p.arr("B", [[3.0]])
    p.mm("A", "B", "C")
    p.check("C", exact=True)


@probe
def p89_shapeop_output_then_chain(p):
    M, N = 16, 24
    p.randn("X", M, N)
    p.t("X", "Xt")
    p.rs("Xt", (N, M), "Xt_flat")
    p.ew("mul", "t", "Xt_flat", 2.0)
    p.ew("exp", "y", "t")
    p.check("y")


@probe
def p90_reduction_with_prologue_then_epilogue(p):
    p.randn("X", 16, 32)
    p.ew("mul", "X1", "X", 2.0)
    p.red("sum", "s", "X1")
    p.ew("mul", "s1", "s", 0.5)
    p.ew("exp", "y", "s1")
    p.check("y")


@probe
def p91_matmul_output_to_reduction(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.red("sum", "rs", "C")
    p.check("rs")


@probe
def p92_reduction_then_two_chain_consumers_both_anchors(p):
    M = 32
    p.randn("X", M, 32)
    p.randn("Y", M, 32)
    p.randn("Z", M, 32)
    p.red("sum", "rs", "X")
    p.rs("rs", (M, 1), "rs2d")
    p.ew("add", "A", "Y", "rs2d", y="col")
    p.ew("mul", "B", "Z", "rs2d", y="col")
    p.check("A", "B")


@probe
def p93_chain_reads_view_of_reduction_output(p):
    M = 16
    p.randn("X", M, 32)
    p.red("sum", "rs", "X")
    p.rs("rs", (M, 1), "rs_col")
    p.rs("rs", (1, M), "rs_row")
    p.arr("O", np.ones((M, M)))
    p.ew("add", "t", "O", "rs_col", y="col")
    p.ew("add", "y", "t", "rs_row", y="row")
    p.check("y")


@probe
def p94_shape_op_then_reduction(p):
    M, N = 8, 16
    p.randn("X", M, N)
    p.t("X", "Xt")
    p.rs("Xt", (N, M), "Xt_flat")
    p.red("sum", "rs", "Xt_flat")
    p.check("rs")


@probe
def p95_elementwise_chain_with_first_op_unary_then_binary_tensor(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("exp", "t1", "X")
    p.ew("add", "t2", "t1", "Y")
    p.check("t2")


@probe
def p96_chain_intermediate_is_program_output(p):
    p.randn("X", 16, 32)
    p.ew("add", "t1", "X", 1.0)
    p.ew("mul", "t2", "t1", 2.0)
    p.check("t2", exact=True)


@probe
def p98_reduction_intermediate_is_program_output(p):
    p.randn("X", 16, 32)
    p.red("sum", "s", "X")
    p.ew("mul", "y", "s", 2.0)
    p.check("y")


@probe
def p99_elementwise_shape_1_1(p):
    p.arr("X", [[2.5]])
    p.ew("mul", "y", "X", 3.0)
    p.check("y", exact=True)


# ---------------------------------------------------------------------------
# p100 .. p129
# ---------------------------------------------------------------------------


@probe
def p100_where_then_chain(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.arr("Cond", p.rng.standard_normal((16, 32)) > 0)
    p.ew("where", "w", "X", "Y", "Cond")
    p.ew("mul", "z", "w", 0.5)
    p.check("z", exact=True)


@probe
def p101_two_kernels_share_input_then_consume_each_other(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("add", "t1", "X", "Y")
    p.ew("mul", "t2", "t1", "X")
    p.check("t2", exact=True)


@probe
def p102_unary_chain_then_unary_chain(p):
    p.arr("X", np.abs(p.rng.standard_normal((16, 32))).astype(F32) + F32(0.1))
    p.ew("exp", "a", "X")
    p.ew("sqrt", "b", "a")
    p.ew("log", "y", "b")
    p.check("y")


@probe
def p103_reduction_then_op_then_back_reduction(p):
    M = 16
    p.randn("X", M, 32)
    p.red("sum", "rs", "X")
    p.ew("mul", "m", "rs", 2.0)
    p.rs("m", (M, 1), "m2d")
    p.red("sum", "final", "m2d")
    p.check("final")


@probe
def p104_transpose_then_transpose_then_op(p):
    p.randn("X", 16, 24)
    p.randn("Y", 16, 24)
    p.t("X", "Xt")
    p.t("Xt", "Xtt")
    p.ew("add", "z", "Xtt", "Y")
    p.check("z", exact=True)


@probe
def p105_chain_where_in_middle_of_chain(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.arr("Cond", p.rng.standard_normal((16, 32)) > 0)
    p.ew("add", "a", "X", 1.0)
    p.ew("where", "b", "a", "Y", "Cond")
    p.ew("mul", "c", "b", 2.0)
    p.check("c", exact=True)


@probe
def p106_matmul_then_two_reductions(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.red("max", "rmax", "C")
    p.red("min", "rmin", "C")
    p.check("rmax", "rmin")


@probe
def p107_negate_of_comparison(p):
    p.randn("X", 16, 32)
    p.ew("gt", "mask", "X", 0.0)
    p.ew("negate", "y", "mask")
    p.check("y", exact=True)


@probe
def p108_div_by_zero_handling(p):
    p.arr("X", [[1.0, -1.0, 2.0, 0.0, -2.0, 3.0, -3.0, 4.0],
                [-4.0, 5.0, -5.0, 6.0, -6.0, 7.0, -7.0, 8.0],
                [-8.0, 9.0, -9.0, 10.0, -10.0, 11.0, -11.0, 12.0],
                [1e30, -1e30, 1e-30, -1e-30, 0.0, 0.0, 0.0, 0.0]])
    z = np.zeros((4, 8), F32)
    z[0, 3] = 1.0
    z[3, 4] = 1.0
    p.arr("Y", np.where(z == 0, 0.5, z))
    p.ew("div", "z", "X", "Y")
    p.check("z", exact=True)


@probe
def p109_input_used_only_via_view(p):
    p.randn("X", 16, 32)
    p.randn("Y", 32, 16)
    p.t("X", "Xt")
    p.ew("add", "z", "Y", "Xt")
    p.check("z", exact=True)


@probe
def p110_chain_with_two_consumers_one_is_view(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("add", "t1", "X", "Y")
    p.rs("t1", (16, 32), "t1_v")
    p.ew("mul", "t2", "t1", 3.0)
    p.check("t2", exact=True)


@probe
def p111_matmul_output_with_strided_consumer(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.randn("D", 32, 32)
    p.mm("A", "B", "C")
    p.t("C", "Ct")
    p.ew("add", "z", "D", "Ct")
    p.check("z")


@probe
def p112_recompute_with_comparison_op(p):
    p.randn("X", 32, 32)
    p.randn("B1", 32, 32)
    p.randn("B2", 32, 32)
    p.ew("gt", "mask", "X", 0.0)
    p.mm("mask", "B1", "t1")
    p.mm("mask", "B2", "t2")
    p.check("t1", "t2")


@probe
def p113_matmul_register_epilogue_with_comparison(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.ew("gt", "mask", "C", 0.0)
    p.check("mask")


@probe
def p114_reduce_then_min_with_negate(p):
    p.randn("X", 16, 32)
    p.red("min", "rm", "X")
    p.ew("negate", "y", "rm")
    p.check("y", exact=True)


@probe
def p115_two_matmul_aliased_through_reshape(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.randn("D", 32, 32)
    p.mm("A", "B", "C")
    p.rs("C", (32, 32), "C_view")
    p.mm("C_view", "D", "E")
    p.check("E")


@probe
def p116_diamond_shared_a_via_transpose_view(p):
    p.randn("X", 16, 16)
    p.randn("B1", 16, 16)
    p.randn("B2", 16, 16)
    p.t("X", "Xt")
    p.mm("Xt", "B1", "t1")
    p.mm("Xt", "B2", "t2")
    p.ew("add", "out", "t1", "t2")
    p.check("out")


@probe
def p117_diamond_with_a_distinct_names_same_buffer(p):
    p.randn("X", 16, 16)
    p.randn("B1", 16, 16)
    p.randn("B2", 16, 16)
    p.rs("X", (16, 16), "X_v1")
    p.rs("X", (16, 16), "X_v2")
    p.mm("X_v1", "B1", "t1")
    p.mm("X_v2", "B2", "t2")
    p.ew("add", "out", "t1", "t2")
    p.check("out")


@probe
def p118_elementwise_output_as_input_to_another_with_view(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("mul", "t1", "X", 2.0)
    p.rs("t1", (16, 32), "t1_v")
    p.ew("add", "y", "t1_v", "Y")
    p.check("y", exact=True)


@probe
def p119_chain_with_scalar_first_then_tensor(p):
    p.randn("X", 32, 32)
    p.randn("Y", 32, 32)
    p.randn("B", 32, 32)
    p.ew("mul", "t1", "X", 2.0)
    p.ew("add", "t2", "t1", "Y")
    p.mm("t2", "B", "C")
    p.check("C")


@probe
def p120_elementwise_chain_5_ops_with_intermediate_outputs(p):
    p.randn("X", 8, 16)
    p.ew("add", "a", "X", 1.0)
    p.ew("mul", "b", "a", 2.0)
    p.ew("max", "c", "b", 0.0)
    p.ew("exp", "d", "c")
    p.ew("log", "e", "d")
    p.check("e")


@probe
def p121_multi_producer_comparison_merge(p):
    p.randn("A1", 16, 16)
    p.randn("B1", 16, 16)
    p.randn("A2", 16, 16)
    p.randn("B2", 16, 16)
    p.mm("A1", "B1", "t1")
    p.mm("A2", "B2", "t2")
    p.ew("gt", "mask", "t1", "t2")
    p.check("mask")


@probe
def p122_chain_fuse_across_named_consumer(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("add", "t1", "X", 1.0)
    p.ew("add", "y", "Y", "t1")
    p.check("y", exact=True)


@probe
def p123_reduce_epilogue_comparison_with_negate(p):
    p.randn("X", 16, 32)
    p.red("sum", "s", "X")
    p.ew("gt", "y", "s", 0.0)
    p.ew("negate", "z", "y")
    p.check("z")


@probe
def p124_matmul_aligned_with_register_epilogue_chain_4_ops(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.mm("A", "B", "z")
    p.ew("add", "z1", "z", 1.0)
    p.ew("mul", "z2", "z1", 0.5)
    p.ew("max", "z3", "z2", 0.0)
    p.ew("exp", "y", "z3")
    p.check("y")


@probe
def p125_dispatch_chain_with_consecutive_kernels_sharing_input(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("add", "a", "X", "Y")
    p.ew("mul", "b", "a", "X")
    p.ew("add", "c", "b", "X")
    p.check("c", exact=True)


@probe
def p126_reduce_along_axis_then_immediately_use_via_view(p):
    M = 16
    p.randn("X", M, 32)
    p.red("sum", "rs", "X")
    p.rs("rs", (M, 1), "rs_col")
    p.randn("Y", M, M)
    p.ew("mul", "z", "Y", "rs_col", y="col")
    p.check("z")


@probe
def p127_long_chain_register_epilogue_relu_sequence(p):
    p.randn("A", 64, 64)
    p.randn("B", 64, 64)
    p.mm("A", "B", "z")
    cur = "z"
    for i in range(10):
        p.ew("max", f"r{i}", cur, 0.0)
        cur = f"r{i}"
    p.check("r9")


@probe
def p128_multi_anchor_followed_by_epilogue(p):
    for n in ("A1", "B1", "A2", "B2"):
        p.randn(n, 16, 16)
    p.mm("A1", "B1", "t1")
    p.mm("A2", "B2", "t2")
    p.ew("add", "merged", "t1", "t2")
    p.ew("max", "out", "merged", 0.0)
    p.check("out")


@probe
def p129_multi_anchor_with_prologue_into_either_anchor(p):
    p.randn("X", 16, 16)
    p.randn("B1", 16, 16)
    p.randn("B2", 16, 16)
    p.ew("max", "X1", "X", 0.0)
    p.mm("X1", "B1", "t1")
    p.mm("X", "B2", "t2")
    p.ew("add", "out", "t1", "t2")
    p.check("out")


# ---------------------------------------------------------------------------
# p200 .. p266: op coverage, small-K matmuls, boundary and IEEE cases
# ---------------------------------------------------------------------------

_FLOOR_CEIL_X = [[0.0, 0.5, 0.9, 1.0, 1.1, -0.1, -0.5, -0.9],
                 [-1.0, -1.1, 2.7, -2.7, 100.3, -100.3, 1e6, -1e6],
                 [0.001, -0.001, 0.999, -0.999, 3.5, -3.5, 7.0, -7.0],
                 [0.0, -0.0, 1.5, -1.5, 2.0, -2.0, 0.4, -0.4]]


@probe
def p200_absolute_op(p):
    p.reseed(42)
    x = p.rng.standard_normal((16, 32)).astype(F32)
    x[0, :4] = [0.0, -0.0, -1e20, 1e20]
    p.arr("X", x)
    p.ew("absolute", "y", "X")
    p.check("y", exact=True)


@probe
def p201_floor_op(p):
    p.arr("X", _FLOOR_CEIL_X)
    p.ew("floor", "y", "X")
    p.check("y", exact=True)


@probe
def p202_ceil_op(p):
    p.arr("X", _FLOOR_CEIL_X)
    p.ew("ceil", "y", "X")
    p.check("y", exact=True)


def _trig(p, op):
    x = p.rng.uniform(-np.pi, np.pi, (16, 32)).astype(F32)
    x[0, 0] = 0.0
    p.arr("X", x)
    p.ew(op, "y", "X")
    p.check("y")


@probe
def p203_sin_op(p):
    _trig(p, "sin")


@probe
def p204_cos_op(p):
    _trig(p, "cos")


@probe
def p205_ge_comparison(p):
    x = p.rng.standard_normal((16, 32)).astype(F32)
    x[0, :2] = 0.0
    p.arr("X", x)
    p.ew("ge", "mask", "X", 0.0)
    p.check("mask", exact=True)


@probe
def p206_le_comparison(p):
    x = p.rng.standard_normal((16, 32)).astype(F32)
    x[0, :2] = [0.0, 1.0]
    p.arr("X", x)
    p.ew("le", "mask", "X", 0.0)
    p.check("mask", exact=True)


@probe
def p207_binary_min_op(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("min", "z", "X", "Y")
    p.check("z", exact=True)


def _small_k(p, M, K, N):
    p.randn("A", M, K)
    p.randn("B", K, N)
    p.mm("A", "B", "C")
    p.check("C")


@probe
def p208_matmul_k1(p):
    _small_k(p, 64, 1, 64)


@probe
def p209_matmul_k2(p):
    _small_k(p, 64, 2, 64)


@probe
def p210_floor_then_chain(p):
    p.uniform("X", -5.0, 5.0, 16, 32)
    p.ew("floor", "f", "X")
    p.ew("mul", "f2", "f", 2.0)
    p.ew("add", "y", "f2", 1.0)
    p.check("y", exact=True)


@probe
def p211_product_reduction_with_single_zero(p):
    x = p.rng.uniform(0.5, 2.0, (16, 32)).astype(F32)
    x[0::2, 0] = 0.0
    p.arr("X", x)
    p.red("product", "p", "X")
    p.check("p")


@probe
def p212_ge_le_boundary_exact_equal(p):
    x = p.randn("X", 16, 32)
    p.arr("Y", x.copy())
    p.ew("ge", "ge_mask", "X", "Y")
    p.ew("le", "le_mask", "X", "Y")
    p.check("ge_mask", "le_mask", exact=True)


@probe
def p213_absolute_in_matmul_epilogue(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.ew("absolute", "y", "C")
    p.check("y")


@probe
def p214_floor_as_matmul_prologue(p):
    p.uniform("X", -3.0, 3.0, 32, 32)
    p.randn("B", 32, 32)
    p.ew("floor", "Xf", "X")
    p.mm("Xf", "B", "C")
    p.check("C")


@probe
def p215_ge_then_sum_count_positive(p):
    p.randn("X", 32, 64)
    p.ew("ge", "mask", "X", 0.0)
    p.red("sum", "count", "mask")
    p.check("count", exact=True)


@probe
def p216_le_broadcast_row(p):
    p.randn("X", 16, 32)
    p.randn("thresh", 1, 32)
    p.ew("le", "mask", "X", "thresh", y="row")
    p.check("mask", exact=True)


@probe
def p217_matmul_k3(p):
    _small_k(p, 32, 3, 32)


@probe
def p218_sin_cos_identity(p):
    p.uniform("X", -np.pi, np.pi, 16, 32)
    p.ew("sin", "s", "X")
    p.ew("cos", "c", "X")
    p.ew("mul", "s2", "s", "s")
    p.ew("mul", "c2", "c", "c")
    p.ew("add", "one", "s2", "c2")
    p.check("one")


@probe
def p219_ceil_then_reduce(p):
    p.uniform("X", -3.0, 3.0, 16, 48)
    p.ew("ceil", "cx", "X")
    p.red("max", "row_max", "cx")
    p.check("row_max", exact=True)


@probe
def p220_ge_not_le_direction(p):
    p.arr("X", [[1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0],
                [-1.0, -2.0, 0.0, 5.0, 5.0, 4.9, 5.1, 10.0],
                [5.0] * 8,
                [0.0, 1.0, 2.0, 3.0, 4.0, 6.0, 7.0, 8.0]])
    p.ew("ge", "ge_mask", "X", 5.0)
    p.ew("le", "le_mask", "X", 5.0)
    p.check("ge_mask", "le_mask", exact=True)


@probe
def p221_ge_single_consumer_matmul_prologue(p):
    p.randn("X", 32, 32)
    p.randn("B", 32, 32)
    p.ew("ge", "mask", "X", 0.0)
    p.mm("mask", "B", "C")
    p.check("C")


@probe
def p222_le_in_matmul_register_epilogue(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.ew("le", "mask", "C", 0.0)
    p.check("mask")


@probe
def p223_floor_in_reduction_epilogue(p):
    p.uniform("X", -5.0, 5.0, 16, 32)
    p.red("sum", "s", "X")
    p.ew("floor", "y", "s")
    p.check("y")


@probe
def p224_abs_in_reduction_prologue(p):
    p.randn("X", 32, 64)
    p.ew("absolute", "aX", "X")
    p.red("sum", "s", "aX")
    p.check("s")


@probe
def p225_matmul_k4(p):
    _small_k(p, 32, 4, 32)


@probe
def p226_matmul_k8(p):
    _small_k(p, 32, 8, 32)


@probe
def p227_product_reduction_large_k(p):
    p.uniform("X", 0.98, 1.02, 8, 256)
    p.red("product", "p", "X")
    p.check("p")


@probe
def p228_ge_chain_into_reduce(p):
    p.randn("X", 32, 64)
    p.ew("ge", "mask", "X", 0.0)
    p.ew("mul", "xpos", "mask", "X")
    p.red("sum", "s", "xpos")
    p.check("s")


@probe
def p229_reduction_k4(p):
    p.randn("X", 16, 4)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p230_floor_of_negative_integers(p):
    p.arr("X", [[-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0, 4.0],
                [-10.0, -5.0, -4.0, -3.5, 3.5, 4.0, 5.0, 10.0],
                [-0.0, 0.0, -1.5, 1.5, -2.5, 2.5, -7.0, 7.0],
                [-100.0, 100.0, -0.001, 0.001, -99.9, 99.9, -50.5, 50.5]])
    p.ew("floor", "y", "X")
    p.check("y", exact=True)


@probe
def p231_ge_two_tensors_no_broadcast(p):
    p.randn("X", 16, 32)
    p.randn("Y", 16, 32)
    p.ew("ge", "mask", "X", "Y")
    p.check("mask", exact=True)


@probe
def p232_abs_then_ge_then_sum(p):
    p.randn("X", 32, 64)
    p.ew("absolute", "aX", "X")
    p.ew("ge", "mask", "aX", 1.0)
    p.red("sum", "count", "mask")
    p.check("count", exact=True)


@probe
def p233_ceil_in_register_epilogue(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.mm("A", "B", "C")
    p.ew("ceil", "y", "C")
    p.check("y")


@probe
def p234_matmul_k5_prime(p):
    _small_k(p, 32, 5, 32)


@probe
def p235_le_col_broadcast(p):
    p.randn("X", 16, 32)
    p.randn("thresh", 16, 1)
    p.ew("le", "mask", "X", "thresh", y="col")
    p.check("mask", exact=True)


@probe
def p236_scalar_literal_tiny_positive(p):
    p.randn("X", 16, 32)
    p.ew("add", "y", "X", 1e-40)
    p.check("y", exact=True)


@probe
def p237_where_then_reduce(p):
    p.randn("X", 32, 64)
    p.randn("Y", 32, 64)
    p.arr("Cond", p.rng.standard_normal((32, 64)) > 0)
    p.ew("where", "W", "X", "Y", "Cond")
    p.red("sum", "s", "W")
    p.check("s")


@probe
def p238_multiple_reductions_same_input(p):
    p.randn("X", 16, 64)
    p.red("sum", "s1", "X")
    p.red("max", "s2", "X")
    p.red("min", "s3", "X")
    p.check("s1")
    p.check("s2", "s3", exact=True)


@probe
def p239_matmul_k16(p):
    _small_k(p, 32, 16, 32)


@probe
def p240_matmul_k17(p):
    _small_k(p, 32, 17, 32)


@probe
def p241_negate_ge_negate_chain(p):
    p.randn("X", 16, 32)
    p.ew("negate", "nx", "X")
    p.ew("ge", "mask", "nx", 0.0)
    p.ew("negate", "nmask", "mask")
    p.check("nmask", exact=True)


@probe
def p242_ge_as_prologue_into_reduction(p):
    p.randn("X", 32, 64)
    p.ew("ge", "mask", "X", 0.0)
    p.red("sum", "s", "mask")
    p.check("s", exact=True)


@probe
def p243_matmul_K256(p):
    _small_k(p, 64, 256, 64)


@probe
def p244_reduction_K256(p):
    p.randn("X", 16, 256)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p245_reduction_K512(p):
    p.randn("X", 8, 512)
    p.red("sum", "s", "X")
    p.check("s")


@probe
def p246_ge_in_tg_tile_matmul_epilogue(p):
    p.randn("A", 32, 32)
    p.randn("B", 32, 32)
    p.randn("bias", 1, 32)
    p.mm("A", "B", "C")
    p.ew("add", "Cb", "C", "bias", y="row")
    p.ew("ge", "mask", "Cb", 0.0)
    p.check("mask")


@probe
def p247_large_matmul_256x256(p):
    _small_k(p, 256, 64, 256)


@probe
def p248_floor_then_absolute(p):
    p.uniform("X", -3.0, 3.0, 16, 32)
    p.ew("floor", "f", "X")
    p.ew("absolute", "y", "f")
    p.check("y", exact=True)


@probe
def p249_reduce_product_K128(p):
    p.uniform("X", 0.99, 1.01, 8, 128)
    p.red("product", "p", "X")
    p.check("p")


@probe
def p250_reduce_product_K129(p):
    p.uniform("X", 0.99, 1.01, 8, 129)
    p.red("product", "p", "X")
    p.check("p")


@probe
def p251_scalar_inf_as_min_clamp(p):
    p.reseed(42)
    p.randn("X", 16, 16)
    p.ew("min", "y", "X", float("inf"))
    p.check("y", exact=True)


@probe
def p252_scalar_neg_inf_as_max_clamp(p):
    p.reseed(42)
    p.randn("X", 16, 16)
    p.ew("max", "y", "X", float("-inf"))
    p.check("y", exact=True)


@probe
def p255_equal_nan_self(p):
    p.arr("X", np.full((8, 8), np.nan))
    p.ew("equal", "mask", "X", float("nan"))
    p.check("mask", exact=True)


@probe
def p256_not_equal_nan_self(p):
    p.arr("X", np.full((8, 8), np.nan))
    p.ew("not_equal", "mask", "X", float("nan"))
    p.check("mask", exact=True)


@probe
def p257_mul_zero_by_inf(p):
    p.arr("X", np.zeros((8, 8)))
    p.arr("INF", np.full((8, 8), np.inf))
    p.ew("mul", "y", "X", "INF")
    p.check("y", exact=True)


@probe
def p259_recip_of_inf(p):
    p.arr("X", np.full((8, 8), np.inf))
    p.ew("recip", "y", "X")
    p.check("y", exact=True)


@probe
def p260_log_of_zero(p):
    p.arr("X", np.zeros((8, 8)))
    p.ew("log", "y", "X")
    p.check("y", exact=True)


@probe
def p265_reduce_sum_with_nan_input(p):
    p.arr("X", [[np.nan, 1.0, 2.0, 3.0], [4.0, 5.0, 6.0, 7.0]])
    p.red("sum", "r", "X")
    p.check("r", exact=True)


@probe
def p266_where_operand_is_nan_tensor(p):
    p.arr("cond", [[1.0, 0.0, 1.0, 0.0]] * 4)
    p.arr("x", np.full((4, 4), np.nan))
    p.arr("y", np.ones((4, 4)))
    p.ew("where", "out", "x", "y", "cond")
    p.check("out", exact=True)


# ---------------------------------------------------------------------------
# The reference's end-to-end scenarios (runner.py:200-415), compared there
# with MLX at rtol = 1e-3, atol = 1e-2 (runner.py:87-102).
# ---------------------------------------------------------------------------

SCENARIOS: dict[str, Callable[[Probe], None]] = {}


def scenario(fn: Callable[[Probe], None]) -> Callable[[Probe], None]:
    SCENARIOS[fn.__name__] = fn
    return fn


def build_scenario(name: str) -> Probe:
    p = Probe()
    SCENARIOS[name](p)
    return p


def _dense_relu(p, x: str, w: str, b: str, out: str, tag: str) -> None:
    p.mm(x, w, f"z{tag}")
    p.ew("add", f"z{tag}b", f"z{tag}", b, y="row")
    p.ew("max", out, f"z{tag}b", 0.0)


@scenario
def s1_big_matmul_aligned(p):
    p.randn("A", 1024, 1024)
    p.randn("B", 1024, 1024)
    p.mm("A", "B", "C")
    p.check("C")


@scenario
def s2_mlp_layer(p):
    p.randn("X", 512, 512)
    p.randn("W", 512, 512)
    p.randn("bias", 1, 512)
    p.mm("X", "W", "z")
    p.ew("add", "zb", "z", "bias", y="row")
    p.ew("max", "y", "zb", 0.0)
    p.check("y")


@scenario
def s3_gelu_chain(p):
    """tanh-form GELU on a matmul output: 0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3)))."""
    p.randn("A", 512, 512)
    p.randn("B", 512, 512)
    p.mm("A", "B", "z")
    p.ew("mul", "z2", "z", "z")
    p.ew("mul", "z3", "z2", "z")
    p.ew("mul", "zc", "z3", 0.044715)
    p.ew("add", "zs", "z", "zc")
    p.ew("mul", "zk", "zs", float(np.sqrt(2.0 / np.pi)))
    p.ew("tanh", "zt", "zk")
    p.ew("add", "z1", "zt", 1.0)
    p.ew("mul", "zh", "z", 0.5)
    p.ew("mul", "y", "zh", "z1")
    p.check("y")


@scenario
def s4_diamond_multi_consumer(p):
    p.randn("A", 256, 256)
    p.randn("B", 256, 256)
    p.mm("A", "B", "t")
    p.ew("max", "r", "t", 0.0)
    p.ew("exp", "e", "t")
    p.check("r", "e")


@scenario
def s5_attention_block(p):
    S = 128
    p.randn("Q", S, 64)
    p.randn("Kmat", S, 64)
    p.randn("V", S, 64)
    p.t("Kmat", "Kt")
    p.mm("Q", "Kt", "scores")
    p.red("max", "row_max", "scores")
    p.rs("row_max", (S, 1), "row_max_2d")
    p.ew("subtract", "shifted", "scores", "row_max_2d", y="col")
    p.ew("exp", "num", "shifted")
    p.red("sum", "row_sum", "num")
    p.rs("row_sum", (S, 1), "row_sum_2d")
    p.ew("div", "probs", "num", "row_sum_2d", y="col")
    p.mm("probs", "V", "out")
    p.check("out")


@scenario
def s6_layernorm_like(p):
    M, N = 256, 512
    p.randn("X", M, N)
    p.red("sum", "row_sum", "X")
    p.ew("mul", "mean", "row_sum", 1.0 / N)
    p.rs("mean", (M, 1), "mean_2d")
    p.ew("subtract", "centered", "X", "mean_2d", y="col")
    p.ew("mul", "sq", "centered", "centered")
    p.red("sum", "sq_sum", "sq")
    p.ew("mul", "var", "sq_sum", 1.0 / N)
    p.ew("add", "var_eps", "var", 1e-5)
    p.ew("sqrt", "std", "var_eps")
    p.rs("std", (M, 1), "std_2d")
    p.ew("div", "y", "centered", "std_2d", y="col")
    p.check("y")


@scenario
def s7_nonaligned_matmul(p):
    p.randn("A", 257, 129)
    p.randn("B", 129, 193)
    p.randn("bias", 1, 193)
    p.mm("A", "B", "z")
    p.ew("add", "zb", "z", "bias", y="row")
    p.ew("max", "y", "zb", 0.0)
    p.check("y")


@scenario
def s8_tall_skinny_matmul(p):
    p.randn("A", 4096, 64)
    p.randn("B", 64, 4096)
    p.mm("A", "B", "C")
    p.check("C")


@scenario
def s9_stacked_mlps(p):
    p.randn("X", 256, 256)
    p.randn("W1", 256, 512)
    p.randn("b1", 1, 512)
    p.randn("W2", 512, 256)
    p.randn("b2", 1, 256)
    _dense_relu(p, "X", "W1", "b1", "h1", "1")
    _dense_relu(p, "h1", "W2", "b2", "y", "2")
    p.check("y")


@scenario
def s10_many_tensor_operands(p):
    for i in range(6):
        p.randn(f"x{i}", 256, 256)
    prev = "x0"
    for i, out in enumerate(("s1", "s2", "s3", "s4", "y"), start=1):
        p.ew("add", out, prev, f"x{i}")
        prev = out
    p.check("y", exact=True)
