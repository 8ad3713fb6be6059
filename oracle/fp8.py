"""fp8 e4m3fn arithmetic of the KV path, restated in numpy (oracle; tests only).

Follows ``_fp8_roundtrip`` at wavelet/trainer/models/deepseek_v4/attention.py:41-50:

    scale = exp2(ceil(log2(amax.clamp_min(1e-10) / 448)))
    q     = (x / scale).clamp(-448, 448).to(float8_e4m3fn)
    x_hat = q.float() * scale

``e4m3_encode`` reproduces torch's fp32 -> float8_e4m3fn cast bit for bit (RNE,
no saturation: a value that rounds above 448 becomes the NaN code 0x7F with
the sign kept), which is why the clamp comes first. ``pow2_scale`` evaluates
``ceil(log2(.))`` exactly with frexp instead of libm's log2.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
AMAX_FLOOR = np.float32(1e-10)  # attention.py:45 clamp_min(1e-10)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn codes (uint8), bit-identical to torch's ``.to(float8_e4m3fn)``."""
    f = np.asarray(x, dtype=np.float32)
    bits = f.view(np.uint32)
    sign = ((bits >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    with np.errstate(invalid="ignore"):
        a = np.abs(f).astype(np.float64)
    code = np.zeros(f.shape, dtype=np.int64)

    sub = a < 2.0**-6
    code[sub] = np.rint(a[sub] * 512.0).astype(np.int64)  # multiples of 2^-9, RNE

    nrm = ~sub & np.isfinite(a)
    mant, exp = np.frexp(a[nrm])  # a = mant * 2^exp, mant in [0.5, 1)
    e = exp.astype(np.int64) - 1  # a = (2*mant) * 2^e, 2*mant in [1, 2)
    q = np.rint(mant * 16.0).astype(np.int64)  # 1.xxx with 3 fraction bits, in [8, 16]
    code[nrm] = ((e + 7) << 3) + (q - 8)  # a carry out of the mantissa bumps the exponent

    code = np.where(np.isnan(f) | np.isinf(f) | (code >= 0x7F), 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    """e4m3fn codes -> exact fp32 values (0x7F / 0xFF decode to NaN)."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0**-9, (8 + m) * np.exp2(e.astype(np.float64) - 10.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def pow2_scale(amax: np.ndarray) -> np.ndarray:
    """Smallest power of two >= max(amax, 1e-10) / 448, as fp32 (attention.py:42-48).

    ``amax`` is clamped into [1e-10, FLT_MAX] first (an infinite amax saturates
    to FLT_MAX so the block still has a finite scale); the fp32 division
    ``a / 448`` is IEEE-rounded like torch's, and ``ceil(log2(.))`` is exact.
    """
    a = np.asarray(amax, dtype=np.float32)
    a = np.minimum(np.maximum(a, AMAX_FLOOR), np.float32(np.finfo(np.float32).max))
    r = (a / np.float32(E4M3_MAX)).astype(np.float32)
    mant, exp = np.frexp(r.astype(np.float64))  # r = mant * 2^exp, mant in [0.5, 1)
    e = np.where(mant == 0.5, exp - 1, exp)  # exact power of two: ceil(log2 r) = exp - 1
    return np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)


def quantize(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``e4m3(clamp(x / scale, -448, 448))`` as attention.py:49 does it (fp32 math)."""
    with np.errstate(invalid="ignore", divide="ignore"):  # NaN / inf inputs are part of the domain
        v = np.asarray(x, dtype=np.float32) / np.asarray(scale, dtype=np.float32)
    v = np.where(np.isnan(v), v, np.clip(v, -E4M3_MAX, E4M3_MAX)).astype(np.float32)
    return e4m3_encode(v)


def dequantize(code: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``code.float() * scale`` (attention.py:50; dequantize.py:45-62)."""
    return (e4m3_decode(code) * np.asarray(scale, dtype=np.float32)).astype(np.float32)
