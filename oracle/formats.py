"""Packed formats and quantizers restated in numpy.

Each function follows the reference line range it names.  Integers are held
as int64 so no step can overflow; words are reported as int32 bit patterns.
"""

from __future__ import annotations

import numpy as np

from .numerics import FP8_MAX, e4m3_decode, e4m3_encode

# kairyu/quant/awq.py:14-15 -- nibble i of a packed word holds column ORDER[i]
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _to_i32(words: np.ndarray) -> np.ndarray:
    return (np.asarray(words, dtype=np.int64) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def _u32(words) -> np.ndarray:
    return np.asarray(words).astype(np.int64) & 0xFFFFFFFF


# ---------------------------------------------------------------- AWQ
def awq_pack(values) -> np.ndarray:
    """kairyu/quant/awq.py:18-25: [rows, cols] -> int32 [rows, cols//8]."""

    v = np.asarray(values, dtype=np.int64) & 0xF
    rows, cols = v.shape
    words = np.zeros((rows, cols // 8), dtype=np.int64)
    for nibble, column in enumerate(AWQ_ORDER):
        words |= v[:, column::8] << (4 * nibble)
    return _to_i32(words)


def awq_unpack(packed) -> np.ndarray:
    """kairyu/quant/awq.py:28-36: int32 [rows, cols//8] -> int64 [rows, cols]."""

    w = _u32(packed)
    rows, pcols = w.shape
    out = np.zeros((rows, pcols * 8), dtype=np.int64)
    for nibble, column in enumerate(AWQ_ORDER):
        out[:, column::8] = (w >> (4 * nibble)) & 0xF
    return out


def awq_dequantize(qweight, qzeros, scales, group_size: int) -> np.ndarray:
    """kairyu/quant/awq.py:62-74 -> fp32 [out, in], w = (q - z) * s."""

    q = awq_unpack(qweight).astype(np.float32)
    z = awq_unpack(qzeros).astype(np.float32)
    s = np.asarray(scales, dtype=np.float32)
    g = np.arange(q.shape[0]) // group_size
    return np.ascontiguousarray(((q - z[g]) * s[g]).T)


# --------------------------------------------------------------- GPTQ
def gptq_pack_rows(values) -> np.ndarray:
    """kairyu/quant/gptq.py:15-21: LSB-first along rows -> int32 [rows//8, cols]."""

    v = np.asarray(values, dtype=np.int64) & 0xF
    rows, cols = v.shape
    words = np.zeros((rows // 8, cols), dtype=np.int64)
    for nibble in range(8):
        words |= v[nibble::8, :] << (4 * nibble)
    return _to_i32(words)


def gptq_unpack_rows(packed) -> np.ndarray:
    w = _u32(packed)
    rows8, cols = w.shape
    out = np.zeros((rows8 * 8, cols), dtype=np.int64)
    for nibble in range(8):
        out[nibble::8, :] = (w >> (4 * nibble)) & 0xF
    return out


def gptq_pack_cols(values) -> np.ndarray:
    """kairyu/quant/gptq.py:32-38: LSB-first along columns -> int32 [rows, cols//8]."""

    v = np.asarray(values, dtype=np.int64) & 0xF
    rows, cols = v.shape
    words = np.zeros((rows, cols // 8), dtype=np.int64)
    for nibble in range(8):
        words |= v[:, nibble::8] << (4 * nibble)
    return _to_i32(words)


def gptq_unpack_cols(packed) -> np.ndarray:
    w = _u32(packed)
    rows, pcols = w.shape
    out = np.zeros((rows, pcols * 8), dtype=np.int64)
    for nibble in range(8):
        out[:, nibble::8] = (w >> (4 * nibble)) & 0xF
    return out


def gptq_dequantize(qweight, qzeros, scales, g_idx) -> np.ndarray:
    """kairyu/quant/gptq.py:78-90 -> fp32 [out, in], w = (q - (z_stored + 1)) * s[g_idx]."""

    q = gptq_unpack_rows(qweight).astype(np.float32)
    z = (gptq_unpack_cols(qzeros) + 1).astype(np.float32)
    s = np.asarray(scales, dtype=np.float32)
    g = np.asarray(g_idx, dtype=np.int64)
    return np.ascontiguousarray(((q - z[g]) * s[g]).T)


def w4a16_weight_fp16(w_fp32_products: np.ndarray) -> np.ndarray:
    """The kernel contract rounds each dequantized weight to fp16
    (quant_gemm_gpu.py:294, 385): returns float32 holding fp16 values."""

    return np.asarray(w_fp32_products, dtype=np.float32).astype(np.float16).astype(np.float32)


# ---------------------------------------------------------------- INT8
def int8_quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """kairyu/quant/int8.py:17-30: s = max(amax, 1e-12)/127 (fp32),
    q = clamp(round_half_even(x/s), +-127)."""

    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1, keepdims=True)
    scale = np.maximum(amax, np.float32(1e-12)) / np.float32(127.0)
    q = np.clip(np.rint(x / scale), -127, 127).astype(np.int8)
    return q, scale.astype(np.float32)


# ----------------------------------------------------------------- FP8
def fp8_quantize_rows(x, static_scale=None) -> tuple[np.ndarray, np.ndarray]:
    """kairyu/quant/fp8.py:33-45: dynamic s = max(amax, 1e-12)/448 per row, or a
    static scalar; q = e4m3(clamp(x/s, +-448)).  Returns (uint8 bytes, fp32 scale)."""

    x = np.asarray(x, dtype=np.float32)
    if static_scale is None:
        amax = np.abs(x).max(axis=-1, keepdims=True)
        scale = np.maximum(amax, np.float32(1e-12)) / np.float32(FP8_MAX)
    else:
        scale = np.full(x.shape[:-1] + (1,), np.float32(static_scale), dtype=np.float32)
    q = e4m3_encode(np.clip(x / scale, -FP8_MAX, FP8_MAX))
    return q, scale.astype(np.float32)


def fp8_quantize_weight(w, per_channel: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """kairyu/quant/fp8.py:20-30 on fp32 weights [out, in]."""

    w = np.asarray(w, dtype=np.float32)
    if per_channel:
        amax = np.abs(w).max(axis=1, keepdims=True)
    else:
        amax = np.abs(w).max().reshape(1)
    scale = (np.maximum(amax, np.float32(1e-12)) / np.float32(FP8_MAX)).astype(np.float32)
    q = e4m3_encode(np.clip(w / scale, -FP8_MAX, FP8_MAX))
    return q, scale


def fp8_dequantize(bits, scale) -> np.ndarray:
    return e4m3_decode(bits) * np.asarray(scale, dtype=np.float32)


# ------------------------------------------------------------ block FP8
BLOCK = 128


def block_fp8_quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """Per row, per 128-wide K block: s = max(amax_blk, 1e-12)/448 (fp32),
    q = e4m3(clamp(x/s, +-448)) -- kairyu/quant/fp8.py:33-45 applied blockwise."""

    x = np.asarray(x, dtype=np.float32)
    rows, k = x.shape
    nb = -(-k // BLOCK)
    scales = np.empty((rows, nb), dtype=np.float32)
    q = np.empty((rows, k), dtype=np.uint8)
    for b in range(nb):
        sl = slice(b * BLOCK, min(k, (b + 1) * BLOCK))
        amax = np.abs(x[:, sl]).max(axis=1, keepdims=True)
        s = np.maximum(amax, np.float32(1e-12)) / np.float32(FP8_MAX)
        scales[:, b : b + 1] = s
        q[:, sl] = e4m3_encode(np.clip(x[:, sl] / s, -FP8_MAX, FP8_MAX))
    return q, scales


def block_fp8_quantize_weight(w) -> tuple[np.ndarray, np.ndarray]:
    """128x128 blocks of w [out, in]: s = max(amax, 1e-12)/448, q = e4m3(clamp(w/s))."""

    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    nb, kb = -(-n // BLOCK), -(-k // BLOCK)
    scales = np.empty((nb, kb), dtype=np.float32)
    q = np.empty((n, k), dtype=np.uint8)
    for i in range(nb):
        for j in range(kb):
            rs = slice(i * BLOCK, min(n, (i + 1) * BLOCK))
            cs = slice(j * BLOCK, min(k, (j + 1) * BLOCK))
            amax = np.float32(np.abs(w[rs, cs]).max())
            s = np.maximum(amax, np.float32(1e-12)) / np.float32(FP8_MAX)
            scales[i, j] = s
            q[rs, cs] = e4m3_encode(np.clip(w[rs, cs] / s, -FP8_MAX, FP8_MAX))
    return q, scales


def block_fp8_dequantize(bits, scales) -> np.ndarray:
    v = e4m3_decode(bits)
    n, k = v.shape
    s = np.repeat(np.repeat(np.asarray(scales, np.float32), BLOCK, 0), BLOCK, 1)[:n, :k]
    return v * s
