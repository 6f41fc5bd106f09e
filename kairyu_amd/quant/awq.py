"""AWQ W4A16 checkpoint format ("gemm" layout).

Interface of kairyu/quant/awq.py:14-74.  Storage:

* ``qweight`` int32 ``[in, out // 8]``: nibble ``i`` (bits ``4i..4i+3``) of
  packed column ``j`` holds original column ``8j + AWQ_ORDER[i]``.
* ``qzeros`` int32 ``[in // g, out // 8]``, packed the same way.
* ``scales`` fp16 ``[in // g, out]``.
* Dequantization ``w = (q - z) * s`` (no +1 offset; that is GPTQ's).
"""

from __future__ import annotations

import torch

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)

def _shifts(device) -> torch.Tensor:
    return torch.arange(0, 32, 4, dtype=torch.int64, device=device)


def pack_awq(values: torch.Tensor) -> torch.Tensor:
    """int values ``[rows, cols]`` (``cols % 8 == 0``) -> int32 ``[rows, cols // 8]``."""

    rows, cols = values.shape
    if cols % 8:
        raise ValueError(f"AWQ packing needs cols % 8 == 0, got {cols}")
    octets = values.to(torch.int64).reshape(rows, cols // 8, 8) & 0xF
    nibbles = octets[:, :, list(AWQ_ORDER)]  # nibble i <- column ORDER[i]
    words = (nibbles << _shifts(nibbles.device)).sum(dim=-1)  # disjoint bit fields
    return words.to(torch.int32)


def unpack_awq(packed: torch.Tensor) -> torch.Tensor:
    """int32 ``[rows, cols // 8]`` -> int32 ``[rows, cols]`` in original column order."""

    rows, packed_cols = packed.shape
    wide = packed.to(torch.int64) & 0xFFFFFFFF
    nibbles = (wide.unsqueeze(-1) >> _shifts(wide.device)) & 0xF  # [rows, pc, 8] nibble order
    columns = nibbles[:, :, list(AWQ_REVERSE_ORDER)]  # column c <- nibble REVERSE[c]
    return columns.reshape(rows, packed_cols * 8).to(torch.int32)


def quantize_awq(
    weight: torch.Tensor, group_size: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric min/max per group along ``in``.

    ``weight [out, in]`` -> ``(qweight [in, out//8], qzeros [in//g, out//8],
    scales fp16 [in//g, out])``: ``s = max(max - min, 1e-5) / 15``,
    ``z = clamp(round(-min / s), 0, 15)``, ``q = clamp(round(w / s) + z, 0, 15)``.
    """

    out_features, in_features = weight.shape
    if in_features % group_size:
        raise ValueError("AWQ in_features must be divisible by group_size")
    groups = in_features // group_size
    w = weight.to(torch.float32).t().reshape(groups, group_size, out_features)
    low = w.amin(dim=1)
    high = w.amax(dim=1)
    scales = (high - low).clamp(min=1e-5) / 15.0
    zeros = torch.round(-low / scales).clamp(0, 15)
    q = (torch.round(w / scales.unsqueeze(1)) + zeros.unsqueeze(1)).clamp(0, 15)
    q = q.reshape(in_features, out_features).to(torch.int32)
    return pack_awq(q), pack_awq(zeros.to(torch.int32)), scales.to(torch.float16)


def dequantize_awq(
    qweight: torch.Tensor,
    qzeros: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
) -> torch.Tensor:
    """-> fp32 weight ``[out, in]`` (``nn.Linear`` layout)."""

    q = unpack_awq(qweight).to(torch.float32)
    zeros = unpack_awq(qzeros).to(torch.float32)
    group = torch.arange(q.shape[0], device=q.device) // group_size
    w = (q - zeros[group]) * scales.to(torch.float32)[group]
    return w.t().contiguous()
