"""The whole-output matmul checker (``tests/matmul_check.py``) on the CPU:
it accepts float32 products summed the ways the GPU kernels sum them
(32-wide k-chunks, chunk ranges split between workgroups and added
afterwards, any chunk order) and rejects the mistakes a tile walk or a
stream-K hand-over could make -- a zeroed tile, a dropped or duplicated
k-chunk of one tile, two tiles swapped, one 32x32 MFMA block missing a
chunk -- each planted in a CPU-computed result."""

from __future__ import annotations

import numpy as np
import pytest

from tests.matmul_check import accumulation_bound, check_matmul, check_matmul_product

TK, TILE = 32, 256


def _chunked(a: np.ndarray, b: np.ndarray, order=None) -> np.ndarray:
    """float32 A @ B accumulated one 32-wide k-chunk at a time in float32."""
    K = a.shape[1]
    chunks = list(range(K // TK)) if order is None else order
    c = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for k in chunks:
        c += a[:, k * TK : (k + 1) * TK] @ b[k * TK : (k + 1) * TK]
    return c


def _operands(M=512, K=1024, N=768, seed=5):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((K, N)).astype(np.float32))


def _chunk(a, b, k, rows, cols):
    return a[rows, k * TK : (k + 1) * TK] @ b[k * TK : (k + 1) * TK, cols]


def test_accepts_fp32_products_in_any_chunk_order_and_split():
    a, b = _operands()
    check_matmul(_chunked(a, b), a, b, "chunked")
    n = a.shape[1] // TK
    check_matmul(_chunked(a, b, order=list(reversed(range(n)))), a, b, "reversed chunks")
    # stream-K: a tile's chunk range split over three workgroups, partial sums added by the owner
    part = [_chunked(a[:, s:e], b[s:e]) for s, e in ((0, 320), (320, 704), (704, 1024))]
    check_matmul((part[0] + part[1]) + part[2], a, b, "split ranges")
    check_matmul(a @ b, a, b, "sgemm")


def test_scale_and_prologue_error_terms():
    a, b = _operands(256, 128, 256)
    s = np.float32(1.0 / np.sqrt(128))
    check_matmul(_chunked(a, b) * s, a, b, "scaled", scale=float(s))
    # A perturbed by up to 2 ulp per element (a bounded-error prologue)
    pert = np.nextafter(np.nextafter(a, np.inf), np.inf)
    check_matmul(_chunked(pert, b), a, b, "perturbed A", a_rel=4 * 2.0**-24)
    with pytest.raises(AssertionError):
        check_matmul(_chunked(a, b), a, b, "unscaled", scale=float(s))


PLANTS = {
    "zeroed tile": lambda c, a, b: c[256:512, 0:256].fill(0.0),
    "dropped chunk": lambda c, a, b: c.__setitem__(
        (slice(0, 256), slice(256, 512)), c[0:256, 256:512] - _chunk(a, b, 5, slice(0, 256), slice(256, 512))
    ),
    "duplicated chunk": lambda c, a, b: c.__setitem__(
        (slice(256, 512), slice(512, 768)), c[256:512, 512:768] + _chunk(a, b, 30, slice(256, 512), slice(512, 768))
    ),
    "swapped tiles": lambda c, a, b: c.__setitem__(
        (slice(0, 256), slice(0, 512)), np.concatenate([c[0:256, 256:512], c[0:256, 0:256]], axis=1)
    ),
    "one MFMA block misses a chunk": lambda c, a, b: c.__setitem__(
        (slice(32, 64), slice(64, 96)), c[32:64, 64:96] - _chunk(a, b, 17, slice(32, 64), slice(64, 96))
    ),
}


@pytest.mark.parametrize("name", sorted(PLANTS))
def test_rejects_planted_tile_mistakes(name):
    a, b = _operands()
    c = _chunked(a, b)
    PLANTS[name](c, a, b)
    with pytest.raises(AssertionError):
        check_matmul(c, a, b, name)


def test_accumulation_bound_catches_a_dropped_chunk_the_stated_bar_mostly_misses():
    """At K = 4096 the stated bar (1e-4 sqrt(K) = 6.4e-3 relative to |A||B|)
    is wider than a 32-term partial sum of N(0, 1) products for most
    elements; 2 gamma_K (4.9e-4) is not."""
    a, b = _operands(256, 4096, 256, seed=6)
    c = _chunked(a, b)
    lost = _chunk(a, b, 77, slice(0, 256), slice(0, 256))
    c -= lost
    mag = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    err = np.abs(lost.astype(np.float64))
    assert np.mean(err > 1e-4 * 64 * mag) < 0.05
    assert np.mean(err > accumulation_bound(4096) * mag) > 0.5
    with pytest.raises(AssertionError):
        check_matmul(c, a, b, "dropped chunk at K = 4096")


def test_diamond_product_check():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((256, 512)).astype(np.float32)
    w1 = rng.standard_normal((512, 256)).astype(np.float32)
    w2 = rng.standard_normal((512, 256)).astype(np.float32)
    z = _chunked(x, w1) * _chunked(x, w2)
    check_matmul_product(z, x, w1, w2, "diamond")
    bad = z.copy()
    bad[:, 128:160] = (_chunked(x, w1) - _chunk(x, w1, 3, slice(None), slice(None)))[:, 128:160] * _chunked(x, w2)[
        :, 128:160
    ]
    with pytest.raises(AssertionError):
        check_matmul_product(bad, x, w1, w2, "diamond, chunk dropped in one accumulator set")
