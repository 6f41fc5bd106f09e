"""Reference forwards of the quantized linear formats (numpy, exact accumulation).

The device contract each kernel must meet, per scheme:

* INT8 (kairyu/quant/linear.py:547-553, int8.py:33-41): activation bytes and
  scales bit-exact; int32 accumulators bit-exact; output
  ``((fp32(acc) * xs) * ws) + bias`` rounded to the activation dtype, bit-exact.
* FP8 (linear.py:463-469, fp8.py:48-56): activation bytes and scales
  bit-exact; ``acc`` is the exact sum of e4m3 products (computed here in fp64,
  where it is exact: products are multiples of 2^-18 below 2^18); output
  ``((acc * xs) * ws) + bias``; device output within 1e-2 normwise.
* W4A16 (quant_gemm_gpu.py:224-407 contract): weights ``fp16((q - z) * s)``,
  activation ``fp16(x)`` (bf16 saturated to +-65504), fp64 dot, ``+ bias``.
"""

from __future__ import annotations

import numpy as np

from . import formats
from .numerics import e4m3_decode, to_dtype, w4a16_activation


def _bias_add(out32: np.ndarray, bias) -> np.ndarray:
    if bias is None:
        return out32
    return (out32 + np.asarray(bias, dtype=np.float32)).astype(np.float32)


def int8_accumulate(x_q, w_q) -> np.ndarray:
    """Exact int32 accumulators.  fp64 BLAS is exact here: every partial sum is
    an integer below 2^53 (|acc| <= K * 127^2)."""

    acc = np.asarray(x_q, np.float64) @ np.asarray(w_q, np.float64).T
    return acc.astype(np.int64)


def int8_forward(x, w_q, w_scale, bias=None, out_dtype="bfloat16"):
    """-> (out float32 holding out_dtype values, x_q, x_scale, acc)."""

    x_q, x_scale = formats.int8_quantize_rows(x)
    acc = int8_accumulate(x_q, w_q)
    ws = np.asarray(w_scale, np.float32).reshape(1, -1)
    out = (acc.astype(np.float32) * x_scale).astype(np.float32) * ws
    out = _bias_add(out.astype(np.float32), bias)
    return to_dtype(out, out_dtype), x_q, x_scale, acc


def fp8_accumulate(x_bits, w_bits) -> np.ndarray:
    """Exact sum of e4m3 products (fp64; exact for K < 2^14 * 2^18 range)."""

    return e4m3_decode(x_bits).astype(np.float64) @ e4m3_decode(w_bits).astype(np.float64).T


def fp8_forward(x, w_bits, w_scale, bias=None, out_dtype="bfloat16", static_scale=None,
                row_scale=None):
    """-> (out, x_bits, x_scale, out_fp32_before_cast)."""

    x = np.asarray(x, np.float32)
    if row_scale is not None:
        scale = np.asarray(row_scale, np.float32).reshape(-1, 1)
        from .numerics import e4m3_encode

        x_bits = e4m3_encode(np.clip(x / scale, -448.0, 448.0))
        x_scale = scale
    else:
        x_bits, x_scale = formats.fp8_quantize_rows(x, static_scale)
    acc = fp8_accumulate(x_bits, w_bits).astype(np.float32)
    ws = np.asarray(w_scale, np.float32).reshape(-1)
    ws = ws.reshape(1, -1) if ws.size > 1 else ws.reshape(1, 1)
    out = ((acc * x_scale).astype(np.float32) * ws).astype(np.float32)
    out = _bias_add(out, bias)
    return to_dtype(out, out_dtype), x_bits, x_scale, out


def w4a16_forward(x, w_dequant_fp32, x_dtype: str, bias=None) -> np.ndarray:
    """``w_dequant_fp32`` is ``(q - z) * s`` in fp32, [out, in]."""

    a = w4a16_activation(x, x_dtype).astype(np.float64)
    w = formats.w4a16_weight_fp16(w_dequant_fp32).astype(np.float64)
    out = (a @ w.T).astype(np.float32)
    out = _bias_add(out, bias)
    return to_dtype(out, x_dtype)


def awq_forward(x, qweight, qzeros, scales, group_size, x_dtype, bias=None) -> np.ndarray:
    w = formats.awq_dequantize(qweight, qzeros, scales, group_size)
    return w4a16_forward(x, w, x_dtype, bias)


def gptq_forward(x, qweight, qzeros, scales, g_idx, x_dtype, bias=None) -> np.ndarray:
    w = formats.gptq_dequantize(qweight, qzeros, scales, g_idx)
    return w4a16_forward(x, w, x_dtype, bias)


def error_metrics(actual, expected) -> dict[str, float]:
    """max-abs, rel-RMSE and the normwise max ratio used by every tolerance."""

    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    diff = a - e
    denom_max = max(float(np.abs(e).max()), 1e-30)
    denom_rms = max(float(np.sqrt(np.mean(e * e))), 1e-30)
    return {
        "max_abs": float(np.abs(diff).max()) if diff.size else 0.0,
        "rel_rmse": float(np.sqrt(np.mean(diff * diff)) / denom_rms) if diff.size else 0.0,
        "normwise_max": float(np.abs(diff).max() / denom_max) if diff.size else 0.0,
    }


def gptq_forward_fast(x, qweight, qzeros, scales, g_idx, x_dtype, bias=None) -> np.ndarray:
    """The reference CPU path's operation order (linear.py:401-404: dequantize to
    fp32, cast to the activation dtype, matmul) with the matmul in fp32 BLAS.
    Used only as the timed CPU baseline; parity checks use ``gptq_forward``."""

    w = formats.w4a16_weight_fp16(formats.gptq_dequantize(qweight, qzeros, scales, g_idx))
    a = w4a16_activation(x, x_dtype)
    out = a @ w.T
    return to_dtype(_bias_add(out.astype(np.float32), bias), x_dtype)


def w4a16_reference(x, w_dequant_fp32, x_dtype: str, bias=None) -> tuple[np.ndarray, np.ndarray]:
    """(pre, abs_terms) of the W4A16 contract: ``pre`` is the fp64 dot of the
    fp16 activation operand and the fp16 weights ``fp16((q - z) * s)`` plus
    the bias, before the cast to ``x_dtype``; ``abs_terms`` is
    ``sum_k |a_k * w_k|`` per output, the scale of any fp32 accumulation error."""

    a = w4a16_activation(x, x_dtype).astype(np.float64)
    w = formats.w4a16_weight_fp16(w_dequant_fp32).astype(np.float64)
    pre = a @ w.T
    if bias is not None:
        pre = pre + np.asarray(bias, np.float32).astype(np.float64)
    return pre, np.abs(a) @ np.abs(w).T


def awq_reference(x, qweight, qzeros, scales, group_size, x_dtype, bias=None):
    return w4a16_reference(x, formats.awq_dequantize(qweight, qzeros, scales, group_size),
                           x_dtype, bias)


def gptq_reference(x, qweight, qzeros, scales, g_idx, x_dtype, bias=None):
    return w4a16_reference(x, formats.gptq_dequantize(qweight, qzeros, scales, g_idx),
                           x_dtype, bias)


def fp8_abs_terms(x_bits, w_bits, x_scale, w_scale) -> np.ndarray:
    """``sum_k |x_k * w_k| * xs * ws`` per output of an FP8 W8A8 product, in
    the output's units (the scale of the fp32 accumulation error)."""

    acc = np.abs(e4m3_decode(x_bits)).astype(np.float64) @ np.abs(e4m3_decode(w_bits)).astype(np.float64).T
    ws = np.asarray(w_scale, np.float64).reshape(-1)
    ws = ws.reshape(1, -1) if ws.size > 1 else ws.reshape(1, 1)
    return acc * np.asarray(x_scale, np.float64).reshape(-1, 1) * ws


def awq_forward_fast(x, qweight, qzeros, scales, group_size, x_dtype, bias=None) -> np.ndarray:
    """AWQ counterpart of ``gptq_forward_fast`` (linear.py:401-404 order, fp32
    BLAS matmul); the timed CPU baseline only."""

    w = formats.w4a16_weight_fp16(formats.awq_dequantize(qweight, qzeros, scales, group_size))
    a = w4a16_activation(x, x_dtype)
    return to_dtype(_bias_add((a @ w.T).astype(np.float32), bias), x_dtype)


def fp8_forward_fast(x_bits, x_scale, w_decoded, w_scale, out_dtype="bfloat16") -> np.ndarray:
    """``fp8_w8a8_matmul`` (kairyu/quant/fp8.py:48-56) in the reference's op
    order -- ``(x_q.f32 @ w_q.f32^T) * x_scale * w_scale`` with an fp32 BLAS
    matmul -- on already quantized rows and an already decoded weight
    (``e4m3_decode``); the timed CPU baseline only (parity uses the exact
    ``fp8_forward``)."""

    acc = e4m3_decode(x_bits) @ np.asarray(w_decoded, np.float32).T
    ws = np.asarray(w_scale, np.float32).reshape(1, -1)
    return to_dtype(((acc * x_scale).astype(np.float32) * ws).astype(np.float32), out_dtype)


def swiglu_reference(gate_pre, up_pre, dtype: str) -> np.ndarray:
    """``silu(gate) * up`` as the reference MLP computes it on fp16 / bf16
    tensors (``kairyu/models/layers.py:243-244``:
    ``down_proj(silu(gate_proj(h)) * up_proj(h))``): the projections' outputs
    are tensors of the activation dtype, torch's silu evaluates
    ``x / (1 + exp(-x))`` in fp32 and rounds, and the product is formed in
    fp32 and rounded.  ``gate_pre`` / ``up_pre``: the projections' values
    before their final cast."""

    g = to_dtype(np.asarray(gate_pre, np.float64).astype(np.float32), dtype).astype(np.float32)
    u = to_dtype(np.asarray(up_pre, np.float64).astype(np.float32), dtype).astype(np.float32)
    with np.errstate(over="ignore"):
        s = to_dtype(g / (np.float32(1.0) + np.exp(-g)), dtype).astype(np.float32)
    return to_dtype(s * u, dtype)
