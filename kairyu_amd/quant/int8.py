"""INT8 W8A8 (compressed-tensors, SmoothQuant-style) format.

Interface of kairyu/quant/int8.py:14-45.  Weights: symmetric int8 with a
per-channel fp32 ``[out, 1]`` scale.  Activations: dynamic per-token symmetric,
``scale = rowmax(|x|) / 127``.  The matmul accumulates exactly in int32 (CPU
``torch.matmul`` has no int8 kernel, so operands are widened to int32).
"""

from __future__ import annotations

import torch

INT8_MAX = 127


def _symmetric_int8(values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    amax = values.abs().amax(dim=-1, keepdim=True).clamp(min=1e-12)
    scale = (amax / INT8_MAX).to(torch.float32)
    q = torch.round(values.to(torch.float32) / scale).clamp(-INT8_MAX, INT8_MAX)
    return q.to(torch.int8), scale


def quantize_int8_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``weight [out, in]`` -> (int8 weight, fp32 scale ``[out, 1]``)."""

    return _symmetric_int8(weight)


def quantize_int8_activation(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [T, in]`` -> (int8 x, fp32 per-token scale ``[T, 1]``)."""

    return _symmetric_int8(x)


def int8_w8a8_matmul(
    x_q: torch.Tensor,
    x_scale: torch.Tensor,
    w_q: torch.Tensor,
    w_scale: torch.Tensor,
) -> torch.Tensor:
    """Exact int32 accumulation, then ``acc * x_scale * w_scale^T`` in fp32."""

    accumulated = torch.matmul(x_q.to(torch.int32), w_q.to(torch.int32).t())
    return accumulated.to(torch.float32) * x_scale * w_scale.t()


def dequantize_int8(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return weight.to(torch.float32) * scale
