"""Canonical arithmetic of the decode funnel (test infrastructure only).

This module is the CPU checker of the MI355X kernels; only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it.

Why a canonical arithmetic.  The reference accumulates BF16 x small-integer
products in FP32 in Tensix FPU order and packs to BF16 before each top-k
(``codegen/coarse_compute.py:109-116``, ``codegen/stage15.py:974-988``,
``codegen/refinement_fusion.py:286-287``).  That order cannot be reproduced
off Tensix, and any order-dependent rounding would let a GPU reduction tree
flip a BF16 score at a top-k cutoff.  The build therefore fixes:

1. Query operands keep the reference's BF16 rounding (q, q15 = bf16(q s / 64),
   qs = bf16(q s / 256)).
2. Each BF16 vector x[256] is represented exactly-or-truncated in fixed
   point: with sig/ex the integer significand and exponent of each element
   (x = sig * 2**ex) and exmax the largest ex of a nonzero element,
   ``X[d] = sign * (sig << (ex - exmax + 14))`` (right shifts truncate toward
   zero), so |X| < 2**22 and x ~= X * 2**fx with ``fx = exmax - 14``.  Elements
   whose exponent is within 14 of the largest one are exact.  |X| < 2**22 is
   what lets the device split X into three signed 8-bit limbs for the int8
   matrix cores.
3. A score's dot product D = sum_d X[d] * c[d] (c the integer key code) is
   computed exactly in int64, so the order of summation is irrelevant.
4. D * 2**(fx + e) is rounded ONCE to FP32 (RNE), then the stage's remaining
   FP32 operations run one at a time with RNE and no fused multiply-add, then
   the result is rounded to BF16 (RNE) as the reference's packer does.
5. Top-k ties at BF16 resolution are broken by the lowest token / centroid
   ID; BF16 values are compared through the order-preserving map
   ``ordered16`` (so -0 sorts just below +0).
"""

from __future__ import annotations

import numpy as np

FX_HEADROOM = 14  # bits below the largest element's LSB kept exactly
X_BOUND = 1 << 22


def bf16_bits(x_f32: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 bit pattern, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x_f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x_f32, dtype=np.float32))
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), out)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def ordered16(bits) -> np.ndarray:
    """Order-preserving map of BF16 bits onto unsigned 16-bit integers."""
    b = np.asarray(bits, dtype=np.uint32)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b ^ 0x8000).astype(np.int64)


def fixed_point(bits: np.ndarray):
    """Fixed-point form of BF16 vectors ``bits`` [..., n] (last axis is one
    vector).  Returns ``(X int64 [..., n], fx int64 [...])`` per rule 2."""
    b = np.asarray(bits, dtype=np.int64)
    expf = (b >> 7) & 0xFF
    mant = b & 0x7F
    sig = np.where(expf == 0, mant, mant | 0x80)
    ex = np.where(expf == 0, -133, expf - 134)
    nonzero = sig != 0
    exmax = np.where(nonzero, ex, -(1 << 20)).max(axis=-1, keepdims=True)
    exmax = np.where(nonzero.any(axis=-1, keepdims=True), exmax, 0)
    shift = ex - exmax + FX_HEADROOM
    mag = np.where(
        shift >= 0,
        sig << np.clip(shift, 0, 62),
        sig >> np.clip(-shift, 0, 62),
    )
    mag = np.where(shift < -62, 0, mag)
    X = np.where(b & 0x8000, -mag, mag)
    return X.astype(np.int64), (exmax[..., 0] - FX_HEADROOM).astype(np.int64)


def exact_dot(X: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """D[..., h, n] = sum_d X[..., h, d] * codes[..., n, d], exactly.

    Every partial sum is an integer below 2**53, so a float64 matmul is exact
    in any summation order (|X| < 2**22, |code| <= 255, 256 terms)."""
    Xf = np.asarray(X, dtype=np.float64)
    Cf = np.asarray(codes, dtype=np.float64)
    D = Xf @ np.swapaxes(Cf, -1, -2)
    return D.astype(np.int64)


def to_f32(D: np.ndarray, exp2: np.ndarray) -> np.ndarray:
    """RNE_f32(D * 2**exp2) for int64 D below 2**53 (rule 4)."""
    v = np.ldexp(np.asarray(D, dtype=np.float64), np.asarray(exp2, dtype=np.int64))
    return v.astype(np.float32)


def sqrt_rne_f32(N: int, fx: int) -> np.float32:
    """RNE_f32(sqrt(N) * 2**fx) for an int64 N >= 0, by integer arithmetic.

    The square root is formed on a left-shifted copy of N so the integer root
    carries at least 26 significant bits; a sticky flag records an inexact
    root, and the 24-bit significand is rounded to nearest even."""
    if N <= 0:
        return np.float32(0.0)
    k = 0
    while N << (2 * (k + 1)) < (1 << 62):
        k += 1
    M = N << (2 * k)
    s = _isqrt(M)
    sticky = s * s != M
    bits = s.bit_length()
    drop = bits - 24
    q = s >> drop
    rem = s & ((1 << drop) - 1)
    half = 1 << (drop - 1)
    if rem > half or (rem == half and (sticky or (q & 1))):
        q += 1
    # value = q * 2**(drop - k + fx)
    return np.float32(np.ldexp(np.float64(q), drop - k + fx))


def _isqrt(n: int) -> int:
    import math

    return math.isqrt(n)


def f32_mul(a, b) -> np.ndarray:
    return (np.asarray(a, dtype=np.float32) * np.asarray(b, dtype=np.float32)).astype(
        np.float32
    )


def f32_add(a, b) -> np.ndarray:
    return (np.asarray(a, dtype=np.float32) + np.asarray(b, dtype=np.float32)).astype(
        np.float32
    )


def f32_sub(a, b) -> np.ndarray:
    return (np.asarray(a, dtype=np.float32) - np.asarray(b, dtype=np.float32)).astype(
        np.float32
    )


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f16_bits_to_bf16_bits(bits) -> np.ndarray:
    """FP16 -> BF16 (exact widening to FP32, then RNE), as torch does."""
    return bf16_bits(f16_to_f32(bits))


def topk_keys(order16: np.ndarray, ids: np.ndarray, id_bits: int) -> np.ndarray:
    """Unique selection keys: larger key = better (score desc, id asc)."""
    return (np.asarray(order16, dtype=np.int64) << id_bits) | (
        ((1 << id_bits) - 1) - np.asarray(ids, dtype=np.int64)
    )


def top_k_by_key(keys: np.ndarray, k: int) -> np.ndarray:
    """Positions of the ``k`` largest unique keys, best first."""
    k = min(k, keys.shape[-1])
    part = np.argpartition(-keys, k - 1)[:k] if k < keys.shape[-1] else np.arange(keys.shape[-1])
    return part[np.argsort(-keys[part], kind="stable")]
