"""INT8 W8A8 device forward under its per-format module name.

Counterpart of the reference's legacy per-format entry
(kairyu/kernels/int8_gemm_gpu.py:8-11): callers that import the format's own
module get the same gfx950 kernel as quant_gemm_hip.int8_linear_forward.
"""

from __future__ import annotations

import torch

from kairyu_amd.kernels.quant_gemm_hip import int8_linear_forward as _forward


def linear_forward(x: torch.Tensor, module) -> torch.Tensor:
    return _forward(x, module)
