"""MoE routing, block-FP8 experts and combine (numpy) -- TEST INFRASTRUCTURE ONLY.

Restates, for the CPU:

* Qwen3 routing, ``kairyu/models/moe.py:255-273``: top-k by a stable
  descending sort of the router logits (ties -> smaller expert id); weights =
  fp32 softmax over the selected logits (``norm_topk_prob``) or the fp32
  softmax over all experts gathered at the selection.
* One SwiGLU expert, ``moe.py:27-83`` with each projection a block-FP8 linear:
  dynamic 1x128 activation blocks and 128x128 weight blocks (the
  ``finegrained_fp8_linear(..., block_size=[128, 128])`` convention the
  reference calls at ``kairyu/kernels/deepseek_v4_moe_gpu.py:60-74``), each
  projection's output rounded to the activation dtype (bf16 or fp16), ``silu``
  and the product rounded to it as torch does for such tensors.
* The combine of ``_mix_experts`` (``moe.py:86-119``) and the EP slot-order
  combine (``moe_parallel.py:255-283``): ``fp32(expert_out) * weight`` summed
  over slots in order in fp32, one final cast.

Block sums are accumulated in float64 (e4m3 products are exact multiples of
2^-18 there), so this is the fp64-accumulated reference the device output is
compared against within a tolerance.
"""

from __future__ import annotations

import numpy as np

from .formats import BLOCK, block_fp8_quantize_rows
from .numerics import e4m3_decode, to_dtype


def softmax_f32(values: np.ndarray) -> np.ndarray:
    """torch.softmax(dtype=float32) restated: exp(v - max) / sum, float32 steps."""

    v = np.asarray(values, dtype=np.float32)
    e = np.exp(v - v.max(axis=-1, keepdims=True)).astype(np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def route_topk(logits, top_k: int, norm_topk_prob: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """(indices int64 [T, k], weights float32 [T, k]) -- moe.py:255-273 (Qwen3)."""

    lg = np.asarray(logits, dtype=np.float32)
    # stable sort of the negated logits == stable descending sort: equal
    # logits keep ascending expert order
    order = np.argsort(-lg, axis=-1, kind="stable")[:, :top_k]
    if norm_topk_prob:
        weights = softmax_f32(np.take_along_axis(lg, order, axis=-1))
    else:
        weights = np.take_along_axis(softmax_f32(lg), order, axis=-1)
    return order.astype(np.int64), weights


def block_gemm(xq, xs, wq, ws) -> np.ndarray:
    """sum over 128-wide K blocks of (qx . qw) * xs[r, b] * ws[n // 128, b], fp64.

    xq uint8 e4m3 [R, K], xs float32 [R, K/128], wq uint8 e4m3 [N, K],
    ws float32 [N/128, K/128] -> float64 [R, N]."""

    xv = e4m3_decode(xq).astype(np.float64)
    wv = e4m3_decode(wq).astype(np.float64)
    rows, k = xv.shape
    n = wv.shape[0]
    out = np.zeros((rows, n), dtype=np.float64)
    wsn = np.repeat(np.asarray(ws, np.float64), BLOCK, axis=0)[:n]  # [N, K/128]
    for b in range(-(-k // BLOCK)):
        sl = slice(b * BLOCK, min(k, (b + 1) * BLOCK))
        part = xv[:, sl] @ wv[:, sl].T  # exact: e4m3 products in fp64
        out += part * np.asarray(xs, np.float64)[:, b : b + 1] * wsn[None, :, b]
    return out


def block_fp8_linear(x, wq, ws, bias=None) -> np.ndarray:
    """One block-FP8 linear on activation-dtype rows: float32 result (before
    the caller's cast).  x [R, K] values, wq [N, K] e4m3 bits, ws [N/128, K/128]."""

    xq, xs = block_fp8_quantize_rows(np.asarray(x, np.float32))
    out = block_gemm(xq, xs, wq, ws).astype(np.float32)
    if bias is not None:
        out = (out + np.asarray(bias, np.float32)).astype(np.float32)
    return out


def silu_f32(v) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    return (v / (np.float32(1.0) + np.exp(-v))).astype(np.float32)


def expert_forward(x, w13q, s13, w2q, s2, dtype: str = "bfloat16") -> np.ndarray:
    """One SwiGLU expert on rows of the activation dtype (``"bfloat16"`` or
    ``"float16"``): gate rows [0, I) and up rows [I, 2I) of the stacked w13
    (grouped_moe.py:144-161); every step rounded to that dtype as the
    reference's expert computes it in torch.  Returns values [R, H]."""

    inter = w13q.shape[0] // 2
    gate_up = block_fp8_linear(x, w13q, s13)
    gate = to_dtype(gate_up[:, :inter], dtype)
    up = to_dtype(gate_up[:, inter:], dtype)
    act = to_dtype(to_dtype(silu_f32(gate), dtype) * up, dtype)
    return to_dtype(block_fp8_linear(act, w2q, s2), dtype)


def combine(expert_out, weights) -> np.ndarray:
    """``out = 0; out = out + fp32(y[:, s]) * w[:, s]`` for s in slot order, in
    float32; y [T, k, H], weights [T, k] -> float32 [T, H] (before the cast)."""

    y = np.asarray(expert_out, dtype=np.float32)
    w = np.asarray(weights, dtype=np.float32)
    out = np.zeros((y.shape[0], y.shape[2]), dtype=np.float32)
    for s in range(y.shape[1]):
        out = (out + (y[:, s, :] * w[:, s : s + 1]).astype(np.float32)).astype(np.float32)
    return out


def moe_forward(hidden, topk_idx, topk_w, w13q, s13, w2q, s2, dtype: str = "bfloat16") -> np.ndarray:
    """Routed block-FP8 experts + slot-order combine.  hidden [T, H] (values
    of ``dtype``), topk_idx [T, k], topk_w [T, k] float32, w13q [E, 2I, H] e4m3
    bits, s13 [E, 2I/128, H/128], w2q [E, H, I], s2 [E, H/128, I/128].
    Returns values of ``dtype`` [T, H]."""

    x = np.asarray(hidden, np.float32)
    idx = np.asarray(topk_idx)
    tokens, top_k = idx.shape
    y = np.zeros((tokens, top_k, x.shape[1]), dtype=np.float32)
    for e in np.unique(idx):
        t, s = np.nonzero(idx == e)
        y[t, s] = expert_forward(x[t], w13q[e], s13[e], w2q[e], s2[e], dtype)
    return to_dtype(combine(y, topk_w), dtype)


def block_fp8_linear_reference(x, wq, ws, bias=None) -> tuple[np.ndarray, np.ndarray]:
    """(pre, abs_terms) of one block-FP8 linear: ``pre`` is the fp64 value
    ``sum_b (qx . qw)_b * xs[r, b] * ws[n // 128, b] (+ bias)`` before any cast;
    ``abs_terms`` the same sum over |qx| and |qw| (the scale of fp32
    accumulation error)."""

    xq, xs = block_fp8_quantize_rows(np.asarray(x, np.float32))
    pre = block_gemm(xq, xs, wq, ws)
    if bias is not None:
        pre = pre + np.asarray(bias, np.float32).astype(np.float64)
    # e4m3 magnitudes: the bits with the sign bit cleared
    abs_terms = block_gemm(np.asarray(xq, np.uint8) & 0x7F, np.abs(xs),
                           np.asarray(wq, np.uint8) & 0x7F, np.abs(ws))
    return pre, abs_terms
