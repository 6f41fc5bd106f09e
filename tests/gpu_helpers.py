"""Helpers shared by the GPU parity tests.

Floating-point outputs are checked per element against the oracle's value
before its final cast (``pre``, accumulated exactly or in fp64):

    |out - pre| <= ulps * ulp_dtype(max(|out|, |pre|))
                   + sqrt(K) * 2^-24 * sum_k |a_k * w_k|     (fp32 accumulation)
                   + 4 * 2^-24 * |pre|                       (epilogue roundings)

One ulp of the output dtype covers the device's final rounding (half an ulp)
plus the part of its fp32 accumulation error that moves the value across a
rounding boundary.  The accumulation slack is ``sqrt(K)`` units of fp32
round-off on the sum of absolute terms: a device that adds ``K/8`` or fewer
partial sums in fp32 stays far inside it, while a dropped or doubled term
(on average ``sum|terms| / K``) exceeds it by a factor ``2^24 / K^1.5``
(64x at K=4096, 9.8x at K=14336) and also exceeds one output ulp on most
outputs (tests/test_parity_bounds.py plants such mistakes in the oracle).
The normwise max error and relative RMSE of the north-star contract (<= 1e-2)
are still computed and reported.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import linear as olinear

DTYPE_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}

# north-star ceiling of the normwise max error and relative RMSE; reported,
# and asserted only where no per-element bound applies
FP_TOL = 1e-2

U32 = 2.0 ** -24
_MANTISSA = {"float16": 10, "bfloat16": 7, "float32": 23}
_EMIN = {"float16": -14, "bfloat16": -126, "float32": -126}


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def ulp(values, dtype: str) -> np.ndarray:
    """Spacing of ``dtype`` numbers at |values| (subnormal spacing below the
    smallest normal)."""

    a = np.abs(np.asarray(values, np.float64))
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(np.where(a > 0, e, _EMIN[dtype]), _EMIN[dtype])
    return np.ldexp(1.0, (e - _MANTISSA[dtype]).astype(np.int64))


def assert_close_fp(actual, expected, tol: float = FP_TOL, label: str = "") -> dict:
    """North-star metrics (normwise max, rel-RMSE) within ``tol``."""

    m = olinear.error_metrics(actual, expected)
    assert m["normwise_max"] <= tol and m["rel_rmse"] <= tol, f"{label} {m}"
    return m


def assert_ulp_close(actual, pre, dtype: str, abs_terms, k: int, label: str = "",
                     ulps: float = 1.0) -> dict:
    """Per-element bound of the module docstring.  ``actual``: device output
    (values of ``dtype``); ``pre``: the oracle's value before the cast;
    ``abs_terms``: the oracle's sum of |terms| per output; ``k``: the
    reduction length.  Prints the histogram of |out - pre| in output ulps."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(pre, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    finite = np.isfinite(ref)
    assert np.array_equal(np.isfinite(out), finite), f"{label}: non-finite pattern differs"
    out, ref = out[finite], ref[finite]
    terms = np.asarray(abs_terms, np.float64)[finite]
    diff = np.abs(out - ref)
    unit = ulp(np.maximum(np.abs(out), np.abs(ref)), dtype)
    bound = ulps * unit + np.sqrt(max(k, 1)) * U32 * terms + 4 * U32 * np.abs(ref)
    ratio = diff / ulp(ref, dtype)
    edges = [0.0, 0.25, 0.5, 0.75, 1.0, 1.5, 2.0, np.inf]
    hist = np.histogram(ratio, bins=edges)[0].tolist() if ratio.size else []
    metrics = olinear.error_metrics(out, ref) if out.size else {}
    metrics.update({"ulp_hist": hist, "max_ulp": float(ratio.max()) if ratio.size else 0.0})
    print(f"[parity] {label} ulp bins {edges[1:-1]}: {hist} max {metrics['max_ulp']:.3f} "
          f"normwise {metrics.get('normwise_max', 0):.3e} rel_rmse {metrics.get('rel_rmse', 0):.3e}",
          flush=True)
    bad = diff > bound
    if bad.any():
        i = int(np.argmax(diff - bound))
        raise AssertionError(
            f"{label}: {int(bad.sum())} of {bad.size} outputs outside {ulps} ulp + "
            f"accumulation slack; worst out={out[i]!r} pre={ref[i]!r} bound={bound[i]!r} {metrics}")
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
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, xd, terms, module.in_features, label)


def check_fp8(out: torch.Tensor, x: torch.Tensor, module, label: str = "", static_scale=None,
              row_scale=None, add_bias: bool = True) -> dict:
    """Per-element check of an FP8 W8A8 device output against the exact
    accumulation ``((acc * xs) * ws) + bias`` before the cast to ``out.dtype``."""

    _, x_bits, x_scale, pre = olinear.fp8_forward(
        np32(x.reshape(-1, x.shape[-1])), bits(module.weight), np32(module.weight_scale),
        _bias_of(module, add_bias), static_scale=static_scale, row_scale=row_scale)
    terms = olinear.fp8_abs_terms(x_bits, bits(module.weight), x_scale, np32(module.weight_scale))
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, DTYPE_NAME[out.dtype], terms,
                            module.in_features, label)


def check_block_fp8(out: torch.Tensor, x: torch.Tensor, module, label: str = "",
                    add_bias: bool = True) -> dict:
    """Per-element check of a dense block-FP8 linear against
    ``sum_b (qx . qw)_b * xs_b * ws_b + bias`` (fp64) before the cast."""

    from oracle import moe as omoe

    pre, terms = omoe.block_fp8_linear_reference(
        np32(x.reshape(-1, x.shape[-1])), bits(module.weight), np32(module.weight_scale_inv),
        _bias_of(module, add_bias))
    return assert_ulp_close(np32(out).reshape(pre.shape), pre, DTYPE_NAME[out.dtype], terms,
                            module.in_features, label)


def assert_moe_close(actual, expected, dtype: str, label: str = "", ulps: float = 2.0,
                     frac: float = 0.99, rel_rmse: float = 3e-3) -> dict:
    """Routed-expert outputs against the oracle's rounded result.

    The expert path rounds twice inside (gate/up to the activation dtype, the
    SwiGLU product re-quantized to e4m3 per 128-wide block), so an fp32
    accumulation difference can move an intermediate across a rounding
    boundary and shift a whole token row by about one output ulp; no
    per-element bound holds for every element.  Asserted instead: at least
    ``frac`` of the outputs within ``ulps`` ulp, and the relative RMSE within
    ``rel_rmse`` (a dropped K term of the 2048-wide gate/up reduction moves it
    to about 2e-2)."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(expected, np.float64)
    diff = np.abs(out - ref)
    ratio = diff / ulp(ref, dtype)
    edges = [0.0, 0.5, 1.0, 2.0, 4.0, 8.0, np.inf]
    hist = np.histogram(ratio, bins=edges)[0].tolist()
    metrics = olinear.error_metrics(out, ref)
    within = float(np.mean(ratio <= ulps))
    metrics.update({"ulp_hist": hist, "within": within})
    print(f"[parity] {label} ulp bins {edges[1:-1]}: {hist} within {ulps} ulp {within:.5f} "
          f"normwise {metrics['normwise_max']:.3e} rel_rmse {metrics['rel_rmse']:.3e}", flush=True)
    assert within >= frac and metrics["rel_rmse"] <= rel_rmse, f"{label} {metrics}"
    return metrics
