"""Helpers shared by the GPU parity tests: device-tensor conversions, the
per-format oracle checks, and assertions over ``oracle.parity``'s criteria
(per-element ulp bound with the MFMA accumulation slack, relative RMSE; the
statistical MoE criterion) -- see that module for the bounds and why."""

from __future__ import annotations

import numpy as np
import torch

from oracle import linear as olinear
from oracle.parity import (  # noqa: F401  (re-exported for the tests)
    U32, e4m3_mfma_slack, fp16_mfma_slack, moe_check, rounding_rel_rmse, swiglu_check, ulp, ulp_check)

DTYPE_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}

# north-star ceiling of the normwise max error and relative RMSE; reported,
# and asserted only where no per-element bound applies
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
    """North-star metrics (normwise max, rel-RMSE) within ``tol``."""

    m = olinear.error_metrics(actual, expected)
    assert m["normwise_max"] <= tol and m["rel_rmse"] <= tol, f"{label} {m}"
    return m


def assert_ulp_close(actual, pre, dtype: str, slack, label: str = "", ulps: float = 1.0,
                     rmse_factor: float = 1.5) -> dict:
    """``oracle.parity.ulp_check`` as an assertion; prints the histogram of
    |out - pre| in output ulps."""

    metrics = ulp_check(actual, pre, dtype, slack, ulps=ulps, rmse_factor=rmse_factor)
    if "ulp_hist" in metrics:
        print(f"[parity] {label} ulp bins {metrics['ulp_bins']}: {metrics['ulp_hist']} "
              f"max {metrics['max_ulp']:.3f} normwise {metrics.get('normwise_max', 0):.3e} "
              f"rel_rmse {metrics['rel_rmse']:.3e} (rounding alone {metrics['rounding_rel_rmse']:.3e})",
              flush=True)
    assert metrics["ok"], f"{label}: {metrics.get('why')} {metrics}"
    return metrics


def banner(text: str) -> None:
    print(f"[gpu-case] {text}", flush=True)


def _bias_of(module, add_bias: bool):
    bias = getattr(module, "bias", None)
    return np32(bias) if (add_bias and bias is not None) else None


def check_w4a16(out: torch.Tensor, module, x: torch.Tensor, label: str = "",
                add_bias: bool = True) -> dict:
    """Per-element check of an AWQ / GPTQ module's device output against
    ``fp64(fp16(x) . fp16((q - z) * s)) + bias`` (the W4A16 kernel contract)."""

    from kairyu_amd.quant.linear import AwqLinear

    xd = DTYPE_NAME[x.dtype]
    xs = np32(x.reshape(-1, x.shape[-1]))
    bias = _bias_of(module, add_bias)
    if isinstance(module, AwqLinear):
        pre, terms = olinear.awq_reference(xs, module.qweight.cpu().numpy(), module.qzeros.cpu().numpy(),
                                           np32(module.scales), module.group_size, xd, bias)
    else:
        pre, terms = olinear.gptq_reference(xs, module.qweight.cpu().numpy(), module.qzeros.cpu().numpy(),
                                            np32(module.scales), module.g_idx.cpu().numpy(), xd, bias)
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, xd,
                            fp16_mfma_slack(terms, module.in_features), label)


def check_fp8(out: torch.Tensor, x: torch.Tensor, module, label: str = "", static_scale=None,
              row_scale=None, add_bias: bool = True) -> dict:
    """Per-element check of an FP8 W8A8 device output against the exact
    accumulation ``((acc * xs) * ws) + bias`` before the cast to ``out.dtype``."""

    from oracle.numerics import e4m3_decode

    w_bits, w_scale = bits(module.weight), np32(module.weight_scale)
    _, x_bits, x_scale, pre = olinear.fp8_forward(
        np32(x.reshape(-1, x.shape[-1])), w_bits, w_scale,
        _bias_of(module, add_bias), static_scale=static_scale, row_scale=row_scale)
    terms = olinear.fp8_abs_terms(x_bits, w_bits, x_scale, w_scale)
    ws = np.abs(w_scale.astype(np.float64)).reshape(-1, 1)
    x_mag = np.abs(e4m3_decode(x_bits)) * np.abs(np.asarray(x_scale, np.float64)).reshape(-1, 1)
    w_mag = np.abs(e4m3_decode(w_bits)) * (ws if ws.size > 1 else ws.reshape(1, 1))
    slack = e4m3_mfma_slack(terms, module.in_features, x_mag, w_mag)
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, DTYPE_NAME[out.dtype], slack, label)


def check_block_fp8(out: torch.Tensor, x: torch.Tensor, module, label: str = "",
                    add_bias: bool = True) -> dict:
    """Per-element check of a dense block-FP8 linear against
    ``sum_b (qx . qw)_b * xs_b * ws_b + bias`` (fp64) before the cast."""

    from oracle import moe as omoe

    from oracle import formats
    from oracle.numerics import e4m3_decode

    xf = np32(x.reshape(-1, x.shape[-1]))
    w_bits, scale_inv = bits(module.weight), np32(module.weight_scale_inv)
    pre, terms = omoe.block_fp8_linear_reference(xf, w_bits, scale_inv, _bias_of(module, add_bias))
    k, n = module.in_features, module.out_features
    xq, xs = formats.block_fp8_quantize_rows(xf)
    x_mag = np.abs(e4m3_decode(xq)) * np.repeat(np.abs(xs), 128, axis=1)[:, :k]
    ws_full = np.repeat(np.repeat(np.abs(scale_inv), 128, axis=0)[:n], 128, axis=1)[:, :k]
    w_mag = np.abs(e4m3_decode(w_bits)) * ws_full
    slack = e4m3_mfma_slack(terms, k, x_mag, w_mag)
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, DTYPE_NAME[out.dtype], slack, label)


def assert_moe_close(actual, expected, dtype: str, label: str = "", **criteria) -> dict:
    """``oracle.parity.moe_check`` as an assertion: the reference's per-element
    tolerance, the normwise maximum, per-row and per-column relative RMSE and
    the whole-tensor statistics of the routed experts."""

    metrics = moe_check(actual, expected, dtype, **criteria)
    print(f"[parity] {label} ulp bins {metrics.get('ulp_bins')}: {metrics.get('ulp_hist')} within "
          f"{metrics.get('within', 0.0):.5f} normwise {metrics.get('normwise_max', 0.0):.3e} "
          f"rel_rmse {metrics.get('rel_rmse', 0.0):.3e} tol ratio {metrics.get('max_tol_ratio', 0.0):.3f} "
          f"row rmse {metrics.get('max_row_rmse', 0.0):.3e} col rmse {metrics.get('max_col_rmse')}",
          flush=True)
    assert metrics["ok"], f"{label} {metrics}"
    return metrics


def projection_pre(module, x: torch.Tensor, add_bias: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """(value before the final cast, accumulation slack) of a quantized
    projection on ``x`` as the oracle computes it: W4A16 and FP8 with their
    MFMA slack, INT8 exact (``((acc * xs) * ws) + bias`` in fp32, no slack)."""

    from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear
    from oracle.numerics import e4m3_decode

    xs = np32(x.reshape(-1, x.shape[-1]))
    bias = _bias_of(module, add_bias)
    xd = DTYPE_NAME[x.dtype]
    if isinstance(module, AwqLinear):
        pre, terms = olinear.awq_reference(xs, module.qweight.cpu().numpy(), module.qzeros.cpu().numpy(),
                                           np32(module.scales), module.group_size, xd, bias)
        return pre, fp16_mfma_slack(terms, module.in_features)
    if isinstance(module, GptqLinear):
        pre, terms = olinear.gptq_reference(xs, module.qweight.cpu().numpy(), module.qzeros.cpu().numpy(),
                                            np32(module.scales), module.g_idx.cpu().numpy(), xd, bias)
        return pre, fp16_mfma_slack(terms, module.in_features)
    if isinstance(module, Int8Linear):
        _, _, x_scale, acc = olinear.int8_forward(xs, module.weight.cpu().numpy(), np32(module.weight_scale),
                                                   None)
        ws = np32(module.weight_scale).reshape(1, -1)
        pre = (acc.astype(np.float32) * x_scale).astype(np.float32) * ws
        if bias is not None:
            pre = (pre + bias.reshape(1, -1)).astype(np.float32)
        return pre.astype(np.float64), np.zeros(pre.shape)
    assert isinstance(module, Fp8Linear)
    w_bits, w_scale = bits(module.weight), np32(module.weight_scale)
    static = None if module.activation_dynamic else np32(module.input_scale)
    _, x_bits, x_scale, pre = olinear.fp8_forward(xs, w_bits, w_scale, bias, static_scale=static)
    terms = olinear.fp8_abs_terms(x_bits, w_bits, x_scale, w_scale)
    ws = np.abs(w_scale.astype(np.float64)).reshape(-1, 1)
    x_mag = np.abs(e4m3_decode(x_bits)) * np.abs(np.asarray(x_scale, np.float64)).reshape(-1, 1)
    w_mag = np.abs(e4m3_decode(w_bits)) * (ws if ws.size > 1 else ws.reshape(1, 1))
    return pre, e4m3_mfma_slack(terms, module.in_features, x_mag, w_mag)


def check_swiglu(out: torch.Tensor, gate, up, x: torch.Tensor, label: str = "") -> dict:
    """``silu(gate(x)) * up(x)`` of a device call against the oracle's
    projections (``oracle.parity.swiglu_check``)."""

    gp, gs = projection_pre(gate, x)
    upre, us = projection_pre(up, x)
    dtype = DTYPE_NAME[out.dtype]
    metrics = swiglu_check(np32(out).reshape(gp.shape), gp, upre, dtype, gs, us)
    print(f"[parity] {label} swiglu ulp bins {metrics.get('ulp_bins')}: {metrics.get('ulp_hist')} "
          f"max {metrics.get('max_ulp', 0):.3f} rel_rmse {metrics.get('rel_rmse', 0):.3e}", flush=True)
    assert metrics["ok"], f"{label}: {metrics.get('why')}"
    return metrics
