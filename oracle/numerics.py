"""Bit-level numerics of the reference's CPU path, restated in numpy.

* ``bf16_round``: torch's float32 -> bfloat16 cast (round to nearest even).
* ``e4m3_encode`` / ``e4m3_decode``: OCP e4m3fn (``torch.float8_e4m3fn``),
  round to nearest even, used after the +-448 clamp the reference applies
  before every fp8 cast (kairyu/quant/fp8.py:29,44).
* ``w4a16_activation``: the W4A16 kernel's activation operand -- fp16 input
  unchanged, bf16 widened and finite values saturated to +-65504 before the
  fp16 cast (kairyu/kernels/quant_gemm_gpu.py:296-307).
"""

from __future__ import annotations

import numpy as np

FP8_MAX = 448.0
FP16_MAX = 65504.0


def bf16_round(values) -> np.ndarray:
    """float32 -> bfloat16 (RNE), returned as float32 holding bf16 values."""

    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = np.isnan(f)
    bits = np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint32) << 16
    return bits.astype(np.uint32).view(np.float32).reshape(f.shape)


def bf16_bits(values) -> np.ndarray:
    return (bf16_round(values).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_bf16(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def fp16_round(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).astype(np.float32)


def to_dtype(values, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ('float16' | 'bfloat16' | 'float32')."""

    if dtype == "float16":
        return fp16_round(values)
    if dtype == "bfloat16":
        return bf16_round(values)
    return np.asarray(values, dtype=np.float32)


def e4m3_encode(values) -> np.ndarray:
    """float32 -> e4m3fn bytes, RNE; |v| >= 448 saturates, NaN -> 0x7f/0xff."""

    v = np.asarray(values, dtype=np.float32)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.minimum(np.abs(v).astype(np.float64), FP8_MAX)
    out = np.zeros(v.shape, dtype=np.uint8)

    sub = a < 2.0**-6
    out[sub] = np.rint(a[sub] * 512.0).astype(np.uint8)  # quantum 2^-9, up to 8

    norm = ~sub & ~np.isnan(a)
    mant, ex = np.frexp(a[norm])  # a = mant * 2**ex, mant in [0.5, 1)
    e = ex - 1  # a = (2*mant) * 2**e
    q = np.rint(mant * 16.0)  # 2*mant*8 in [8, 16]
    carry = q == 16.0
    q = np.where(carry, 8.0, q)
    e = np.where(carry, e + 1, e)
    out[norm] = (((e + 7).astype(np.int64) << 3) | (q.astype(np.int64) - 8)).astype(np.uint8)

    out[np.isnan(v)] = 0x7F
    return out | sign


_E4M3_TABLE = None


def e4m3_decode(bits) -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        table = np.empty(256, dtype=np.float32)
        for b in range(256):
            s = -1.0 if b & 0x80 else 1.0
            e, m = (b >> 3) & 0xF, b & 7
            if e == 15 and m == 7:
                table[b] = np.nan
            elif e == 0:
                table[b] = s * m * 2.0**-9
            else:
                table[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_TABLE = table
    return _E4M3_TABLE[np.asarray(bits, dtype=np.uint8)]


def w4a16_activation(x, dtype: str) -> np.ndarray:
    """Activation operand of the W4A16 dot (float32 array holding fp16 values)."""

    x = np.asarray(x, dtype=np.float32)
    if dtype == "bfloat16":
        finite = np.isfinite(x)
        x = np.where(finite, np.clip(x, -FP16_MAX, FP16_MAX), x)
    return fp16_round(x)
