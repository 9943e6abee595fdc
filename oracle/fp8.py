"""FP8 (OCP E4M3FN / E5M2) and bfloat16 rounding in numpy (test oracle).

Restates the casts the reference relies on:
``scaled.to(torch.float8_e4m3fn)`` (reference ``tcfp/core.py:104``) and
``scaled.to(torch.float8_e5m2)`` (``tcfp/core.py:156``), both
round-to-nearest-even.  Values are pre-clamped to +-FP8_MAX by the
reference, but the encoder also reproduces torch's behaviour just past the
top code (``E4M3``: magnitudes that round above 448 become the NaN code
0x7F, which ``stochastic_round_to_fp8_e4m3`` relies on at
``core.py:452``).
"""
from __future__ import annotations

import numpy as np

E4M3 = "e4m3"
E5M2 = "e5m2"

_FMT = {
    # mantissa bits, exponent bias, max finite, min normal exponent
    E4M3: (3, 7, 448.0, -6),
    E5M2: (2, 15, 57344.0, -14),
}

FP8_MAX = {E4M3: 448.0, E5M2: 57344.0}


def _decode_table(fmt: str) -> np.ndarray:
    mb, bias, _, emin = _FMT[fmt]
    eb = 7 - mb
    out = np.empty(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> mb) & ((1 << eb) - 1)
        m = c & ((1 << mb) - 1)
        if fmt == E4M3 and e == 15 and m == 7:
            v = np.nan
        elif fmt == E5M2 and e == 31:
            v = np.inf if m == 0 else np.nan
        elif e == 0:
            v = m / (1 << mb) * 2.0 ** emin
        else:
            v = (1.0 + m / (1 << mb)) * 2.0 ** (e - bias)
        out[c] = s * v
    return out


DECODE = {E4M3: _decode_table(E4M3), E5M2: _decode_table(E5M2)}


def decode(codes: np.ndarray, fmt: str) -> np.ndarray:
    """uint8 codes -> float32 values."""
    return DECODE[fmt][np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray, fmt: str) -> np.ndarray:
    """float32 -> uint8 codes, round-to-nearest-even (torch CPU cast semantics).

    E4M3FN: magnitudes that round past 448 give 0x7F (NaN), as torch does.
    E5M2: magnitudes that round past 57344 give 0x7C (inf).
    NaN inputs give 0x7F (sign kept).
    """
    mb, bias, _, emin = _FMT[fmt]
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint32)
    mag = bits & np.uint32(0x7FFFFFFF)
    a = mag.view(np.float32)
    # subnormal range: multiples of 2^(emin - mb); a * 2^(mb - emin) is exact
    q_sub = np.rint(a * np.float32(2.0 ** (mb - emin))).astype(np.uint32)
    shift = 23 - mb
    with np.errstate(over="ignore"):
        r = mag + np.uint32((1 << (shift - 1)) - 1) + ((mag >> shift) & np.uint32(1))
    q_norm = (r >> np.uint32(shift)).astype(np.int64) - ((127 - bias) << mb)
    q = np.where(a < np.float32(2.0 ** emin), q_sub.astype(np.int64), q_norm)
    if fmt == E4M3:
        q = np.minimum(q, 0x7F)
    else:
        q = np.minimum(q, 0x7C)
    q = np.where(np.isnan(x), 0x7F, q)
    return (q.astype(np.uint32) | sign).astype(np.uint8)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned widened back to float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    r = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    r = np.where(np.isnan(x), (bits >> 16) | 0x40, r)
    return (r.astype(np.uint32) << 16).view(np.float32)
