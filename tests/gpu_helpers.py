"""Helpers shared by the GPU parity tests.

Floating-point outputs are checked per element against the oracle's value
before its final cast (``pre``, accumulated exactly or in fp64):

    |out - pre| <= ulps * ulp_dtype(max(|out|, |pre|)) + slack + 4 * 2^-24 * |pre|

where the final ulp covers the device's last rounding (half an ulp) plus the
part of its accumulation error that moves the value across a rounding
boundary, ``4 * 2^-24 * |pre|`` the epilogue's fp32 roundings, and ``slack``
the accumulation error of the device's matrix instructions:

* fp16 MFMA (W4A16): ``sqrt(K) * 2^-24 * sum_k |a_k w_k|``, fp32 round-off on
  the sum of absolute terms (the f16 MFMA keeps products down to about 2^-24 of
  the largest product of its group of 8, measured on gfx950);
* e4m3 MFMA (FP8, block FP8): ``2 * (sqrt(K) * 2^-24 * sum_k |a_k w_k| +
  2^-13 * sqrt(7 * sum_g (max_g |a| * max_g |w|)^2))`` in output units.  The
  gfx950 e4m3 MFMA sums each group of 8 products in a window of 13 bits below
  the group's largest product (measured: a product 2^14 below it is dropped);
  the second term is that window's error at a few standard deviations over
  the K/8 groups, with the group maximum bounded by max|a| * max|w|.

A dropped or doubled K term (on average ``sum|terms| / K``) exceeds the slack
on most outputs at the test shapes (tests/test_parity_bounds.py plants such
mistakes in the oracle); at the largest K the relative RMSE check below
catches it as well: every check also requires the relative RMSE of
``out - pre`` to stay within 1.5x of the RMSE of rounding ``pre`` to the
output dtype (a dropped term adds about ``1/sqrt(K)``).
The north-star normwise max error and relative RMSE (<= 1e-2) are reported.
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


def rounding_rel_rmse(pre, dtype: str) -> float:
    """Relative RMSE that rounding ``pre`` to ``dtype`` alone produces
    (uniform error in half an ulp either side: ulp / sqrt(12))."""

    ref = np.asarray(pre, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    if rms == 0.0:
        return 0.0
    return float(np.sqrt(np.mean(ulp(ref, dtype) ** 2) / 12.0)) / rms


def assert_ulp_close(actual, pre, dtype: str, slack, label: str = "", ulps: float = 1.0,
                     rmse_factor: float = 1.5) -> dict:
    """Per-element bound of the module docstring (``slack``: accumulation
    slack per output, output units) plus the relative-RMSE check.  Prints the
    histogram of |out - pre| in output ulps."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(pre, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    finite = np.isfinite(ref)
    assert np.array_equal(np.isfinite(out), finite), f"{label}: non-finite pattern differs"
    out, ref = out[finite], ref[finite]
    slack = np.broadcast_to(np.asarray(slack, np.float64), finite.shape)[finite]
    diff = np.abs(out - ref)
    unit = ulp(np.maximum(np.abs(out), np.abs(ref)), dtype)
    bound = ulps * unit + slack + 4 * U32 * np.abs(ref)
    ratio = diff / ulp(ref, dtype)
    edges = [0.0, 0.25, 0.5, 0.75, 1.0, 1.5, 2.0, np.inf]
    hist = np.histogram(ratio, bins=edges)[0].tolist() if ratio.size else []
    metrics = olinear.error_metrics(out, ref) if out.size else {"rel_rmse": 0.0}
    rounding = rounding_rel_rmse(ref, dtype)
    metrics.update({"ulp_hist": hist, "max_ulp": float(ratio.max()) if ratio.size else 0.0,
                    "rounding_rel_rmse": rounding})
    print(f"[parity] {label} ulp bins {edges[1:-1]}: {hist} max {metrics['max_ulp']:.3f} "
          f"normwise {metrics.get('normwise_max', 0):.3e} rel_rmse {metrics['rel_rmse']:.3e} "
          f"(rounding alone {rounding:.3e})", flush=True)
    bad = diff > bound
    if bad.any():
        i = int(np.argmax(diff - bound))
        raise AssertionError(
            f"{label}: {int(bad.sum())} of {bad.size} outputs outside {ulps} ulp + "
            f"accumulation slack; worst out={out[i]!r} pre={ref[i]!r} bound={bound[i]!r} {metrics}")
    assert metrics["rel_rmse"] <= rmse_factor * rounding + 1e-7, (
        f"{label}: relative RMSE {metrics['rel_rmse']:.3e} above {rmse_factor} x the rounding "
        f"RMSE {rounding:.3e}")
    return metrics


def fp16_mfma_slack(abs_terms, k: int):
    """Accumulation slack of the fp16 MFMA path (module docstring)."""

    return np.sqrt(max(k, 1)) * U32 * np.asarray(abs_terms, np.float64)


def e4m3_mfma_slack(abs_terms, k: int, x_mag, w_mag):
    """Accumulation slack of the e4m3 MFMA path (module docstring).
    ``abs_terms``: sum_k |a_k w_k| in output units; ``x_mag`` [M, K] and
    ``w_mag`` [N, K]: |a| and |w| with their scales applied, so that
    ``x_mag @ w_mag.T`` is in output units too."""

    xm = np.asarray(x_mag, np.float64)
    wm = np.asarray(w_mag, np.float64)
    kk = xm.shape[1]
    pad = (-kk) % 8
    if pad:
        xm = np.pad(xm, ((0, 0), (0, pad)))
        wm = np.pad(wm, ((0, 0), (0, pad)))
    gx = xm.reshape(xm.shape[0], -1, 8).max(axis=2)
    gw = wm.reshape(wm.shape[0], -1, 8).max(axis=2)
    window = 2.0 ** -13 * np.sqrt(7.0 * ((gx * gx) @ (gw * gw).T))
    return 2.0 * (np.sqrt(max(k, 1)) * U32 * np.asarray(abs_terms, np.float64) + window)


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


def assert_moe_close(actual, expected, dtype: str, label: str = "", ulps: float = 8.0,
                     frac: float = 0.95, rel_rmse: float = 5e-3) -> dict:
    """Routed-expert outputs against the oracle's rounded result.

    The expert path rounds inside (gate/up to the activation dtype, the
    SwiGLU product re-quantized to e4m3 per 128-wide block), and its e4m3
    MFMAs sum in a 13-bit window, so an accumulation difference can move an
    intermediate across a rounding boundary and shift a whole token row by a
    few output ulps; no per-element bound holds for every element.  Asserted
    instead: at least ``frac`` of the outputs within ``ulps`` ulp, and the
    relative RMSE within ``rel_rmse`` (a dropped K term of a 2048-wide
    gate/up or 768-wide down reduction moves it to 2-4e-2; measured on
    gfx950 at the test shapes: 0.975-0.997 within 8 ulp, 0.6-2.2e-3)."""

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
