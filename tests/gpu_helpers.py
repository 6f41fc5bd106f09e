"""Helpers shared by the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

from oracle import linear as olinear

DTYPE_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}

# Floating-point tolerance of every non-integer device output versus the
# exact-accumulation oracle: normwise max error and relative RMSE.
FP_TOL = 1e-2


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def assert_close_fp(actual, expected, tol: float = FP_TOL, label: str = "") -> dict:
    m = olinear.error_metrics(actual, expected)
    assert m["normwise_max"] <= tol and m["rel_rmse"] <= tol, f"{label} {m}"
    return m


def banner(text: str) -> None:
    print(f"[gpu-case] {text}", flush=True)
