"""Pins the oracle's canonical arithmetic (``oracle/arith.py``) by means that
do not restate it: exact rational arithmetic, integer brute force and torch's
own casts.  CPU only."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import arith

RNG = np.random.default_rng(20240611)


# ------------------------------------------------------------ independent models
def rne_f32(fr: Fraction) -> float:
    """Round a rational to the nearest FP32 value, ties to even (finite range)."""
    if fr == 0:
        return 0.0
    sign = -1.0 if fr < 0 else 1.0
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 23)
    m = a / quantum
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * float(fl * quantum)


def bf16_value(b: int) -> Fraction:
    return Fraction(float(arith.bf16_to_f32(np.array([b], dtype=np.uint16))[0]))


def all_bf16_finite() -> np.ndarray:
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = arith.bf16_to_f32(b)
    return b[np.isfinite(f)]


# ------------------------------------------------------------------- BF16 / F16
def test_bf16_rounding_matches_torch():
    x = RNG.standard_normal(200_000).astype(np.float32) * np.float32(2.0) ** RNG.integers(
        -140, 120, 200_000
    ).astype(np.float32)
    # exact ties: low 16 bits 0x8000 with both parities of the kept LSB
    ties = (RNG.integers(0, 1 << 16, 4096).astype(np.uint32) << 16) | 0x8000
    ties = ties[np.isfinite(ties.view(np.float32))].view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, -1e-45],
                       dtype=np.float32)
    x = np.concatenate([x, ties, special])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(arith.bf16_bits(x), want)
    nan = arith.bf16_bits(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.isnan(arith.bf16_to_f32(nan)).all()


def test_f16_to_bf16_matches_torch():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = b.view(np.float16)
    ok = ~np.isnan(f)
    want = torch.from_numpy(b.view(np.int16)).view(torch.float16).to(torch.bfloat16)
    want = want.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(arith.f16_bits_to_bf16_bits(b)[ok], want[ok])


def test_ordered16_is_the_value_order():
    b = all_bf16_finite()
    f = arith.bf16_to_f32(b).astype(np.float64)
    o = arith.ordered16(b)
    # sort by value, -0 before +0
    neg_zero = (b == 0x8000)
    order = np.lexsort((~neg_zero, f))
    assert (np.diff(o[order]) > 0).all()
    assert arith.ordered16(np.array([0x8000]))[0] + 1 == arith.ordered16(np.array([0]))[0]


# ---------------------------------------------------------------- fixed point
def _random_bf16_vectors(n, spread):
    x = RNG.standard_normal((n, 256)).astype(np.float32)
    x *= np.float32(2.0) ** RNG.integers(-spread, spread + 1, (n, 256)).astype(np.float32)
    b = arith.bf16_bits(x)
    b[0, :7] = [0, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x7F7F]  # zeros, subnormals, max
    b[1, :] = 0                     # all-zero vector
    b[2, :] = RNG.integers(0, 0x80, 256).astype(np.uint16)  # all subnormal
    return b


@pytest.mark.parametrize("spread", [0, 6, 30])
def test_fixed_point_is_truncation_at_the_stated_scale(spread):
    b = _random_bf16_vectors(12, spread)
    X, fx = arith.fixed_point(b)
    assert (np.abs(X) < arith.X_BOUND).all()
    for r in range(b.shape[0]):
        scale = Fraction(2) ** int(fx[r])
        vals = [bf16_value(int(v)) for v in b[r]]
        for d, v in enumerate(vals):
            assert int(X[r, d]) == int(v / scale), (r, d)  # int() truncates toward 0
        big = max(abs(v) for v in vals)
        if big >= Fraction(2) ** -126:  # a normal element sets the scale
            # the largest element fills 22 bits: a wrong exponent offset fails here
            assert 1 << 21 <= max(abs(int(t)) for t in X[r]) < 1 << 22
            # elements within 14 binades of the largest are exact
            for d, v in enumerate(vals):
                if v != 0 and abs(v) * 2 ** 14 >= big:
                    assert X[r, d] * scale == v


def test_exact_dot_matches_integer_sums_at_the_bound():
    X = RNG.integers(-(1 << 22) + 1, 1 << 22, (4, 256)).astype(np.int64)
    X[0] = (1 << 22) - 1
    X[1] = -(1 << 22) + 1
    c = RNG.integers(0, 256, (37, 256)).astype(np.int64)
    c[0] = 255
    D = arith.exact_dot(X, c)
    for h in range(4):
        for n in range(37):
            assert int(D[h, n]) == sum(int(a) * int(w) for a, w in zip(X[h], c[n]))


def test_to_f32_is_one_rne_rounding():
    D = RNG.integers(-(1 << 52), 1 << 52, 3000).astype(np.int64)
    D[:5] = [0, 1, -1, (1 << 52) - 1, (1 << 24) + 1]
    D[5:500] = (RNG.integers(1 << 23, 1 << 24, 495) * 2 + 1) << RNG.integers(1, 28, 495)
    e = RNG.integers(-80, 20, 3000).astype(np.int64)
    got = arith.to_f32(D, e)
    for i in range(len(D)):
        assert float(got[i]) == rne_f32(Fraction(int(D[i])) * Fraction(2) ** int(e[i])), i


def _sqrt_is_rne(N: int, fx: int, y: np.float32) -> bool:
    V = Fraction(N) * Fraction(2) ** (2 * fx)
    lo = Fraction(float(np.nextafter(y, np.float32(0))))
    hi = Fraction(float(np.nextafter(y, np.float32(np.inf))))
    yv = Fraction(float(y))
    m_lo, m_hi = (lo + yv) / 2, (yv + hi) / 2
    even = (int(np.float32(y).view(np.uint32)) & 1) == 0
    if m_lo * m_lo > V or V > m_hi * m_hi:
        return False
    if V in (m_lo * m_lo, m_hi * m_hi):
        return even
    return True


def test_sqrt_rne_brute_force():
    cases = [(1, 0), (2, 0), (3, -5), (4, 3), (1 << 61, -40), ((1 << 62) - 1, -20)]
    cases += [(int(n), int(f)) for n, f in zip(RNG.integers(1, 1 << 62, 400),
                                               RNG.integers(-60, 10, 400))]
    # exact squares of 25-bit odd integers: the root's 25th bit is a tie
    for s in RNG.integers(1 << 24, 1 << 25, 50) | 1:
        cases.append((int(s) * int(s), -10))
    for N, fx in cases:
        y = arith.sqrt_rne_f32(N, fx)
        assert y > 0 and _sqrt_is_rne(N, fx, y), (N, fx)
    assert arith.sqrt_rne_f32(0, 5) == 0
    assert arith.sqrt_rne_f32(1 << 40, 0) == np.float32(1 << 20)
    assert math.isqrt(99) == 9


# ---------------------------------------------------------------------- top-k
@pytest.mark.parametrize("id_bits", [16, 20])
def test_topk_keys_order_is_score_desc_id_asc(id_bits):
    n = 3000
    scores = arith.bf16_bits(RNG.standard_normal(n).astype(np.float32).round(1))  # many ties
    ids = RNG.permutation(1 << 12)[:n]
    keys = arith.topk_keys(arith.ordered16(scores), ids, id_bits)
    for k in (1, 7, 100, n):
        pos = arith.top_k_by_key(keys, k)
        f = arith.bf16_to_f32(scores).astype(np.float64)
        # value descending, +0 ranked above -0, then the lowest ID
        brute = sorted(range(n), key=lambda i: (-f[i], scores[i] == 0x8000, ids[i]))[:k]
        assert [int(ids[i]) for i in pos] == [int(ids[i]) for i in brute]


# ------------------------------------------------------------------------ FP8
E4M3_GRID = np.array(
    [(m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
     for e in range(16) for m in range(8)][:127]
)  # codes 0x00..0x7e; 0x7f is NaN


def e4m3fn_rne(x: np.ndarray) -> np.ndarray:
    """Value of the e4m3fn code nearest to x (ties to an even code); magnitudes
    past the 448/480 midpoint become NaN."""
    a = np.abs(x)
    idx = np.searchsorted(E4M3_GRID, a)  # grid[idx-1] < a <= grid[idx]
    lo = np.clip(idx - 1, 0, 126)
    hi = np.clip(idx, 0, 126)
    dlo, dhi = a - E4M3_GRID[lo], E4M3_GRID[hi] - a
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    v = E4M3_GRID[pick]
    v = np.where(a > 464.0, np.nan, v)
    return np.copysign(v, x)


def test_fp8_records_rounding_exhaustive_over_bf16():
    from oracle import decode as od

    b = all_bf16_finite()
    k8, v8 = od.fp8_records(b[None, :], b[None, :])
    want = e4m3fn_rne(arith.bf16_to_f32(b).astype(np.float64))
    got = k8[0].astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert np.array_equal(k8, v8, equal_nan=True)
