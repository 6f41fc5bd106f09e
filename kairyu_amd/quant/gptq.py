"""GPTQ W4A16 checkpoint format (v1, "gptq").

Interface of kairyu/quant/gptq.py:15-90.  Storage:

* ``qweight`` int32 ``[in // 8, out]``: sequential, LSB first along ``in``
  (bits ``4i..4i+3`` of word ``r`` hold row ``8r + i``; no reordering).
* ``qzeros`` int32 ``[ceil(in / g), out // 8]``: sequential along ``out``,
  storing ``z - 1``; the +1 is restored at dequantization.
* ``scales`` fp16 ``[ceil(in / g), out]``; ``g_idx`` int32 ``[in]`` maps each
  input row to its group (act-order checkpoints permute it).
* Dequantization ``w = (q - (z_stored + 1)) * s[g_idx]``.
"""

from __future__ import annotations

import torch

def _shifts(device) -> torch.Tensor:
    return torch.arange(0, 32, 4, dtype=torch.int64, device=device)


def _pack_last(nibbles: torch.Tensor) -> torch.Tensor:
    """int64 ``[..., 8]`` nibbles (LSB first) -> int32 words ``[...]``."""

    return ((nibbles & 0xF) << _shifts(nibbles.device)).sum(dim=-1).to(torch.int32)


def _unpack_last(packed: torch.Tensor) -> torch.Tensor:
    """int32 words ``[...]`` -> int64 nibbles ``[..., 8]`` (LSB first)."""

    wide = packed.to(torch.int64) & 0xFFFFFFFF
    return (wide.unsqueeze(-1) >> _shifts(wide.device)) & 0xF


def pack_gptq_rows(values: torch.Tensor) -> torch.Tensor:
    """int ``[rows, cols]`` (``rows % 8 == 0``) -> int32 ``[rows // 8, cols]``."""

    rows, cols = values.shape
    if rows % 8:
        raise ValueError(f"GPTQ row packing needs rows % 8 == 0, got {rows}")
    grouped = values.to(torch.int64).reshape(rows // 8, 8, cols).transpose(1, 2)
    return _pack_last(grouped)


def unpack_gptq_rows(packed: torch.Tensor) -> torch.Tensor:
    rows8, cols = packed.shape
    nibbles = _unpack_last(packed)  # [rows8, cols, 8]
    return nibbles.transpose(1, 2).reshape(rows8 * 8, cols).to(torch.int32)


def pack_gptq_cols(values: torch.Tensor) -> torch.Tensor:
    """int ``[rows, cols]`` (``cols % 8 == 0``) -> int32 ``[rows, cols // 8]``."""

    rows, cols = values.shape
    if cols % 8:
        raise ValueError(f"GPTQ column packing needs cols % 8 == 0, got {cols}")
    return _pack_last(values.to(torch.int64).reshape(rows, cols // 8, 8))


def unpack_gptq_cols(packed: torch.Tensor) -> torch.Tensor:
    rows, packed_cols = packed.shape
    return _unpack_last(packed).reshape(rows, packed_cols * 8).to(torch.int32)


def quantize_gptq(
    weight: torch.Tensor, group_size: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric min/max per group of ``group_size`` consecutive input rows.

    ``weight [out, in]`` -> ``(qweight, qzeros (stored z - 1), scales fp16,
    g_idx = k // group_size)``; the last group may be short.
    """

    out_features, in_features = weight.shape
    groups = -(-in_features // group_size)
    w = weight.to(torch.float32).t().contiguous()  # [in, out]
    g_idx = (torch.arange(in_features) // group_size).to(torch.int32)
    scales = torch.empty(groups, out_features)
    zeros = torch.empty(groups, out_features)
    q = torch.empty(in_features, out_features)
    for group in range(groups):
        lo_row = group * group_size
        hi_row = min(lo_row + group_size, in_features)
        block = w[lo_row:hi_row]
        low = block.amin(dim=0)
        high = block.amax(dim=0)
        scale = (high - low).clamp(min=1e-5) / 15.0
        zero = torch.round(-low / scale).clamp(0, 15)
        scales[group] = scale
        zeros[group] = zero
        q[lo_row:hi_row] = (torch.round(block / scale) + zero).clamp(0, 15)
    stored = (zeros.to(torch.int64) - 1) & 0xF
    return (
        pack_gptq_rows(q.to(torch.int32)),
        pack_gptq_cols(stored),
        scales.to(torch.float16),
        g_idx,
    )


def dequantize_gptq(
    qweight: torch.Tensor,
    qzeros: torch.Tensor,
    scales: torch.Tensor,
    g_idx: torch.Tensor,
    group_size: int,
) -> torch.Tensor:
    """-> fp32 weight ``[out, in]``."""

    del group_size  # the per-row group comes from g_idx
    q = unpack_gptq_rows(qweight).to(torch.float32)
    zeros = (unpack_gptq_cols(qzeros) + 1).to(torch.float32)
    group = g_idx.to(torch.long)
    w = (q - zeros[group]) * scales.to(torch.float32)[group]
    return w.t().contiguous()
