"""The fp32 accumulation of the scans' bf16 MFMAs against exact sums.

The top-k exactness check (merge_refine_kernel), the k-means pick and the
range bounds all rest on one error model of the MFMA accumulator: an
accumulator that chains n products (npass MFMA passes over d elements, the
passes in the scans' order -- rows hi x query plane 0, rows lo x plane 0,
rows hi x plane 1) onto a start value C lies within

    (n + 4) * 2^-23 * S,    S = |C| + sum |a_k b_k|,

of the exact value: one rounding per term at the unit of a truncating fp32
accumulator, which also covers round-to-nearest (2^-24).  This is what keeps
the strict acceptance of TopK.push (index.dart:248-260) exact when the
selection runs on the approximate accumulator.

Each case runs v_mfma_f32_32x32x16_bf16 and v_mfma_f32_16x16x32_bf16 chained
exactly as the scans chain them (vs_dev_mfma_chain), on operands chosen to
stress the accumulator: random data, the split-bf16 planes of fp32 rows and
queries, heavy cancellation, magnitudes spread over 2^-40 .. 2^10, and values
placed a fraction of an ulp from the accumulator.  The exact value is
math.fsum of the products (each exact in fp64: two 8-bit significands).
"""
import ctypes
import math

import numpy as np
import pytest

from vector_store import _native as NN
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu

U23 = 2.0 ** -23
SHAPES = {0: (32, 16), 1: (16, 32)}  # shape: (M = N, K-step)


def bf16(x):
    """bf16 bits of fp32 values, round to nearest even."""
    return syn.to_bf16_bits(np.asarray(x, np.float32))


def f32(bits):
    return syn.bf16_bits_to_f32(bits)


def run(shape, A, B, C):
    """A [npass][M][K], B [npass][N][K] bf16 bits; C [M][N] fp32 -> D."""
    npass, M, K = A.shape
    step = SHAPES[shape][1]
    A = np.ascontiguousarray(A, np.uint16)
    B = np.ascontiguousarray(B, np.uint16)
    C = np.ascontiguousarray(C, np.float32)
    D = np.empty_like(C)
    NN.check(NN.load().vs_dev_mfma_chain(0, shape, K // step, npass,
                                         A.ctypes.data_as(ctypes.c_void_p),
                                         B.ctypes.data_as(ctypes.c_void_p),
                                         C.ctypes.data_as(ctypes.c_void_p),
                                         D.ctypes.data_as(ctypes.c_void_p)))
    return D


def exact(A, B, C):
    """Exact value (math.fsum, correctly rounded to fp64) and S = |C| +
    sum |a b| of every output."""
    a = f32(A).astype(np.float64)  # [p][M][K]
    b = f32(B).astype(np.float64)  # [p][N][K]
    M, N = C.shape
    E = np.empty((M, N))
    S = np.empty((M, N))
    for m in range(M):
        prod = a[:, m:m + 1, :] * b  # [p][N][K], exact
        for n in range(N):
            t = prod[:, n, :].ravel()
            E[m, n] = math.fsum(np.concatenate(([float(C[m, n])], t)))
            S[m, n] = abs(float(C[m, n])) + float(np.abs(t).sum())
    return E, S


def ratio(D, A, B, C):
    """max |D - exact| / ((n + 4) 2^-23 S), n the products per output."""
    E, S = exact(A, B, C)
    n = A.shape[0] * A.shape[2]
    err = np.abs(D.astype(np.float64) - E)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(err > 0, err / ((n + 4) * U23 * S), 0.0)
    return float(r.max())


def case_random(g, M, K):
    A = bf16(g.standard_normal((1, M, K)))
    B = bf16(g.standard_normal((1, M, K)))
    C = g.standard_normal((M, M)).astype(np.float32) * 8
    return A, B, C


def case_planes(g, M, K, l2=True):
    """The scans' three passes: rows x split into hi + lo, queries s q into
    plane 0 + plane 1 (s = -2 for L2), C = the row norms (L2) or 0 (IP)."""
    x = g.standard_normal((M, K)).astype(np.float32)
    q = g.standard_normal((M, K)).astype(np.float32)
    s = -2.0 if l2 else -1.0
    hi = bf16(x)
    lo = bf16(x - f32(hi))
    q0 = bf16(s * q)
    q1 = bf16(s * q - f32(q0))
    A = np.stack([hi, lo, hi])
    B = np.stack([q0, q0, q1])
    xn = (x.astype(np.float64) ** 2).sum(axis=1).astype(np.float32)
    C = np.repeat(xn[:, None], M, axis=1) if l2 else np.zeros((M, M), np.float32)
    return A, B, C


def case_cancel(g, M, K):
    """Large products cancelling pairwise, small ones left over; the start
    value is cancelled by the first products."""
    big = np.exp2(g.integers(4, 10, (1, M, K))).astype(np.float32)
    a = big * (1 + g.integers(0, 127, (1, M, K)) / 128.0)
    b = np.ones((1, M, K), np.float32)
    b[..., 1::2] = -1.0
    a[..., 1::2] = a[..., 0::2]  # exact cancellation in pairs
    small = g.standard_normal((1, M, K)) * 2.0 ** -12
    a[..., 2::8] += small[..., 2::8]
    A = bf16(a)
    B = bf16(b)
    C = (g.standard_normal((M, M)) * 2.0 ** 14).astype(np.float32)
    return A, B, C


def case_mixed(g, M, K):
    ea = g.integers(-20, 6, (1, M, K))
    eb = g.integers(-20, 6, (1, M, K))
    sa = np.where(g.random((1, M, K)) < 0.5, -1.0, 1.0)
    sb = np.where(g.random((1, M, K)) < 0.5, -1.0, 1.0)
    A = bf16(sa * np.exp2(ea) * (1 + g.random((1, M, K))))
    B = bf16(sb * np.exp2(eb) * (1 + g.random((1, M, K))))
    C = (g.standard_normal((M, M)) * 2.0 ** g.integers(-10, 10)).astype(np.float32)
    return A, B, C


def case_near_ulp(g, M, K):
    """C = +-(1 + j ulp) and products a fraction of that ulp: what the
    accumulator keeps of terms below its last bit."""
    j = g.integers(0, 1 << 20, (M, M))
    C = ((1.0 + j * U23) * np.where(g.random((M, M)) < 0.5, -1.0, 1.0)).astype(np.float32)
    frac = g.integers(1, 8, (1, M, K)) / 8.0  # 1/8 .. 7/8 of an ulp of 1
    sgn = np.where(g.random((1, M, K)) < 0.5, -1.0, 1.0)
    A = bf16(sgn * frac * U23)
    B = bf16(np.ones((1, M, K)))
    return A, B, C


CASES = {"random": case_random, "planes_l2": case_planes,
         "planes_ip": lambda g, M, K: case_planes(g, M, K, l2=False),
         "cancel": case_cancel, "mixed": case_mixed, "near_ulp": case_near_ulp}


@pytest.mark.parametrize("shape", [0, 1], ids=["32x32x16", "16x16x32"])
@pytest.mark.parametrize("case", list(CASES))
def test_mfma_accumulation_within_model(vs, shape, case):
    M, step = SHAPES[shape]
    worst = 0.0
    for seed, d in ((1, 768), (2, 256), (3, 128)):
        g = np.random.default_rng([seed, shape, len(case)])
        K = (d // step) * step
        A, B, C = CASES[case](g, M, K)
        D = run(shape, A, B, C)
        assert np.isfinite(D).all()
        worst = max(worst, ratio(D, A, B, C))
    print(f"mfma {['32x32x16', '16x16x32'][shape]} {case}: max error / ((n + 4) 2^-23 S) = "
          f"{worst:.3e}")
    assert worst <= 1.0


@pytest.mark.parametrize("shape", [0, 1], ids=["32x32x16", "16x16x32"])
def test_mfma_layout_and_single_terms(vs, shape):
    """One nonzero product per output lands on the right (row, column), and
    C passes through a chain of zero products unchanged (the lane layout the
    scans assume).  C + a b is not rounded correctly relative to the result
    (measured on gfx950: the terms are aligned to the larger one first, so
    under cancellation the error can exceed half an ulp of the result), but
    it stays within 2^-23 (|C| + |a b|), one unit of the model above."""
    M, step = SHAPES[shape]
    K = 4 * step
    g = np.random.default_rng([7, shape])
    A = np.zeros((1, M, K), np.uint16)
    B = np.zeros((1, M, K), np.uint16)
    a = bf16(np.arange(1, M + 1, dtype=np.float32))
    b = bf16(np.arange(1, M + 1, dtype=np.float32) * 0.5)
    for m in range(M):
        A[0, m, (3 * m) % K] = a[m]
    for n in range(M):
        B[0, n, (3 * n) % K] = b[n]
    C = g.standard_normal((M, M)).astype(np.float32)
    D = run(shape, A, B, C)
    off = ~np.eye(M, dtype=bool)
    assert np.array_equal(D[off], C[off])
    ab = f32(a).astype(np.float64) * f32(b).astype(np.float64)
    c = np.diag(C).astype(np.float64)
    got = np.diag(D).astype(np.float64)
    assert np.all(np.abs(got - (c + ab)) <= U23 * (np.abs(c) + np.abs(ab)))


def test_mfma_rounding_of_sub_ulp_terms(vs):
    """Which way the accumulator rounds terms smaller than its last bit
    (printed for the record; the model above holds either way): C = 1, one
    product of 3/4 ulp(1) -- round to nearest gives 1 + ulp, truncation 1."""
    M, step = SHAPES[0]
    A = np.zeros((1, M, step), np.uint16)
    B = np.zeros((1, M, step), np.uint16)
    A[0, :, 0] = bf16(np.float32(0.75 * U23))
    B[0, :, 0] = bf16(np.float32(1.0))
    C = np.ones((M, M), np.float32)
    D = run(0, A, B, C)
    up = float(D[0, 0]) == 1.0 + U23
    # sixteen products of 1/4 ulp each: one rounding of the exact sum gives
    # 1 + 4 ulp; a rounding after every product leaves 1 (nearest) or 1
    A16 = np.zeros((1, M, step), np.uint16)
    A16[0, :, :] = bf16(np.float32(0.25 * U23))
    B16 = np.zeros((1, M, step), np.uint16)
    B16[0, :, :] = bf16(np.float32(1.0))
    D16 = run(0, A16, B16, C)
    print(f"mfma 32x32x16: 1 + 3/4 ulp -> {'1 + ulp (nearest)' if up else '1 (truncation)'}; "
          f"1 + 16 x 1/4 ulp -> 1 + {(float(D16[0, 0]) - 1.0) / U23:g} ulp")
    assert float(D[0, 0]) in (1.0, 1.0 + U23)
    assert float(D16[0, 0]) in (1.0, 1.0 + U23 * 4, 1.0 + U23 * 3, 1.0 + U23 * 5)
