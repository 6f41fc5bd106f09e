"""Dtype intake of quantized checkpoint tensors.

The loader rule of kairyu/models/loader.py:219-247: a quantized module's
registered buffers are its kernel ABI, so a checkpoint tensor for one of them
is converted to the buffer's own dtype (a bf16-serialized FP8 per-channel
scale becomes fp32, an fp32-serialized W4A16 scale becomes fp16; both
conversions are value-preserving for checkpoint scales), while ordinary fp32
parameters follow the requested compute dtype.  Reading the checkpoint files
is the caller's business; this module only decides dtypes.
"""

from __future__ import annotations

import torch
from torch import nn


def quantized_buffer_dtypes(model: nn.Module) -> dict[str, torch.dtype]:
    """``{state_dict name: dtype}`` of every persistent buffer registered
    directly on a quantized module (``is_quantized``)."""

    dtypes: dict[str, torch.dtype] = {}
    for module_name, module in model.named_modules():
        if not getattr(module, "is_quantized", False):
            continue
        for buffer_name, buffer in module.named_buffers(recurse=False):
            if buffer_name in module._non_persistent_buffers_set:
                continue
            dtypes[f"{module_name}.{buffer_name}" if module_name else buffer_name] = buffer.dtype
    return dtypes


def normalize_quantized_state(model: nn.Module, state: dict[str, torch.Tensor],
                              dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """A copy of ``state`` with quantized buffers in their registered dtype
    and the model's other fp32 floating tensors in ``dtype``."""

    quantized = quantized_buffer_dtypes(model)
    expected = model.state_dict()
    out: dict[str, torch.Tensor] = {}
    for name, tensor in state.items():
        target = quantized.get(name)
        if target is not None and tensor.dtype != target:
            tensor = tensor.to(target)
        elif (target is None and name in expected and expected[name].dtype == torch.float32
              and tensor.is_floating_point()):
            tensor = tensor.to(dtype)
        out[name] = tensor
    return out
