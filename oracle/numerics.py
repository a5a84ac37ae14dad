"""Rounding helpers of the oracle (test infrastructure only).

``round_bf16`` is round-to-nearest-even of fp32/fp64 values to bfloat16, the
rule torch's ``.to(torch.bfloat16)`` applies; ``bf16_round_int`` is the same
rule on exact Python integers/fractions, used to write fixtures without any
floating point in the loop.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np


def round_bf16(a) -> np.ndarray:
    """fp64/fp32 array -> float64 array holding the nearest-even bf16 values.

    fp64 inputs are first rounded to fp32 (as a torch fp32->bf16 cast sees
    them), then to bf16 by integer arithmetic on the fp32 bit pattern.
    Pinned by tests against torch's CPU cast and against ``bf16_round_int``.
    """
    f = np.asarray(a, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def round_fp16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)


def round_fp32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float32).astype(np.float64)


ROUNDERS = {"bf16": round_bf16, "fp16": round_fp16, "fp32": round_fp32}


def bf16_round_int(v) -> Fraction:
    """Exact nearest-even bf16 value of an exact rational (int or Fraction).

    bf16 keeps 8 significant bits; no overflow/underflow handling (fixtures
    stay well inside the normal range).
    """
    v = Fraction(v)
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = 0                      # find e with 2^e <= a < 2^(e+1)
    while a >= 2 ** (e + 1):
        e += 1
    while a < 2 ** e:
        e -= 1
    ulp = Fraction(2) ** (e - 7)
    q, rem = divmod(a, ulp)    # q integer part in ulps
    q = int(q)
    if rem * 2 > ulp or (rem * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp
