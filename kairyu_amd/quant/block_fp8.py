"""128x128 block-scaled FP8 e4m3 format (DeepSeek-style ``weight_block_size``).

The reference has no ``kairyu.quant`` method for it (its detector rejects
``weight_block_size``, kairyu/engine/core/quant_config.py:156-163); its only
block path calls a downloaded hub kernel through
``transformers.integrations.finegrained_fp8.finegrained_fp8_linear(...,
block_size=[128, 128])`` (kairyu/kernels/deepseek_v4_moe_gpu.py:60-74).  This
module fixes the convention that call implies:

* weight e4m3 ``[out, in]`` with ``weight_scale_inv`` fp32
  ``[ceil(out/128), ceil(in/128)]`` and multiplicative dequantization
  ``W[n, k] = q[n, k] * S[n // 128, k // 128]``;
* activations quantized dynamically per token per 128-wide K block,
  ``s = max(amax_block, 1e-12) / 448``, ``q = e4m3(clamp(x / s, +-448))``
  (the per-token formula of kairyu/quant/fp8.py:33-45 applied blockwise).
"""

from __future__ import annotations

import torch

from .fp8 import FP8_MAX

BLOCK = 128


def _blocks(size: int) -> int:
    return -(-size // BLOCK)


def quantize_block_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``weight [..., out, in]`` -> (e4m3 weight, fp32 ``weight_scale_inv [..., ob, ib]``)."""

    *lead, out_features, in_features = weight.shape
    ob, ib = _blocks(out_features), _blocks(in_features)
    w = weight.to(torch.float32)
    padded = torch.zeros(*lead, ob * BLOCK, ib * BLOCK, dtype=torch.float32, device=weight.device)
    padded[..., :out_features, :in_features] = w
    tiles = padded.reshape(*lead, ob, BLOCK, ib, BLOCK)
    amax = tiles.abs().amax(dim=(-3, -1))  # [..., ob, ib]
    scale = (amax.clamp(min=1e-12) / FP8_MAX).to(torch.float32)
    expanded = scale.repeat_interleave(BLOCK, dim=-2).repeat_interleave(BLOCK, dim=-1)
    expanded = expanded[..., :out_features, :in_features]
    q = (w / expanded).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale


def dequantize_block_fp8(weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    out_features, in_features = weight.shape[-2:]
    expanded = scale_inv.to(torch.float32).repeat_interleave(BLOCK, dim=-2)
    expanded = expanded.repeat_interleave(BLOCK, dim=-1)[..., :out_features, :in_features]
    return weight.to(torch.float32) * expanded


def quantize_block_fp8_activation(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [..., in]`` -> (e4m3 ``[..., in]``, fp32 scale ``[..., ceil(in/128)]``)."""

    *lead, in_features = x.shape
    nb = _blocks(in_features)
    xf = x.to(torch.float32)
    padded = torch.zeros(*lead, nb * BLOCK, dtype=torch.float32, device=x.device)
    padded[..., :in_features] = xf
    amax = padded.reshape(*lead, nb, BLOCK).abs().amax(dim=-1)
    scale = (amax.clamp(min=1e-12) / FP8_MAX).to(torch.float32)
    expanded = scale.repeat_interleave(BLOCK, dim=-1)[..., :in_features]
    q = (xf / expanded).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale


def block_fp8_matmul(
    x_q: torch.Tensor,
    x_scale: torch.Tensor,
    w_q: torch.Tensor,
    w_scale_inv: torch.Tensor,
) -> torch.Tensor:
    """Dequantize both operands blockwise, then an fp32 matmul: ``[T, in] x [out, in]^T``."""

    in_features = x_q.shape[-1]
    x = x_q.to(torch.float32) * x_scale.repeat_interleave(BLOCK, dim=-1)[..., :in_features]
    w = dequantize_block_fp8(w_q, w_scale_inv)
    return torch.matmul(x, w.t())
