"""FP8 e4m3 W8A8 (compressed-tensors / "fp8") format.

Interface of kairyu/quant/fp8.py:17-60.  Weights are ``torch.float8_e4m3fn``
with a per-channel ``[out, 1]`` or per-tensor ``(1,)`` fp32 scale; activations
are quantized per token (dynamic) or with a static scalar ``input_scale``.
torch's CPU fp8 cast does not saturate, so values are clamped to +-448 before
the round-to-nearest-even cast.  Every product is computed on upcast values.
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0


def quantize_fp8(
    weight: torch.Tensor, per_channel: bool = True
) -> tuple[torch.Tensor, torch.Tensor]:
    """``weight [out, in]`` -> (e4m3 weight, fp32 scale ``[out, 1]`` or ``(1,)``)."""

    magnitude = weight.abs()
    if per_channel:
        amax = magnitude.amax(dim=1, keepdim=True)
    else:
        amax = magnitude.amax().reshape(1)
    scale = (amax.clamp(min=1e-12) / FP8_MAX).to(torch.float32)
    scaled = (weight.to(torch.float32) / scale).clamp(-FP8_MAX, FP8_MAX)
    return scaled.to(torch.float8_e4m3fn), scale


def quantize_fp8_activation(
    x: torch.Tensor, scale: torch.Tensor | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [..., in]`` -> (e4m3, scale): per-token dynamic, or a static scalar."""

    if scale is None:
        amax = x.abs().amax(dim=-1, keepdim=True).clamp(min=1e-12)
        scale = (amax / FP8_MAX).to(torch.float32)
    elif scale.numel() != 1:
        raise ValueError(f"static FP8 input_scale must be scalar, got {tuple(scale.shape)}")
    else:
        scale = scale.to(device=x.device, dtype=torch.float32)
    scaled = (x.to(torch.float32) / scale).clamp(-FP8_MAX, FP8_MAX)
    return scaled.to(torch.float8_e4m3fn), scale


def fp8_w8a8_matmul(
    x_q: torch.Tensor,
    x_scale: torch.Tensor,
    w_q: torch.Tensor,
    w_scale: torch.Tensor,
) -> torch.Tensor:
    """Upcast reference: ``(x_q @ w_q^T) * x_scale * w_scale`` in fp32."""

    accumulated = torch.matmul(x_q.to(torch.float32), w_q.to(torch.float32).t())
    return accumulated * x_scale * w_scale.reshape(-1)


def dequantize_fp8(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return weight.to(torch.float32) * scale.to(torch.float32)
