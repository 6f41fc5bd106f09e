"""Parity criteria of the device outputs -- TEST INFRASTRUCTURE ONLY.

Used by ``tests/`` and by ``bench.py``'s ``cpu_baseline`` leg to judge a
device output against the oracle's value; nothing in the ``kairyu_amd``
package imports it.

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
mistakes in the oracle); at the largest K the relative RMSE check catches it
as well: every check also requires the relative RMSE of ``out - pre`` to stay
within 1.5x of the RMSE of rounding ``pre`` to the output dtype (a dropped
term adds about ``1/sqrt(K)``).
"""

from __future__ import annotations

import numpy as np

from .linear import error_metrics, swiglu_reference

U32 = 2.0 ** -24
_MANTISSA = {"float16": 10, "bfloat16": 7, "float32": 23}
_EMIN = {"float16": -14, "bfloat16": -126, "float32": -126}


def ulp(values, dtype: str) -> np.ndarray:
    """Spacing of ``dtype`` numbers at |values| (subnormal spacing below the
    smallest normal)."""

    a = np.abs(np.asarray(values, np.float64))
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(np.where(a > 0, e, _EMIN[dtype]), _EMIN[dtype])
    return np.ldexp(1.0, (e - _MANTISSA[dtype]).astype(np.int64))


def rounding_rel_rmse(pre, dtype: str) -> float:
    """Relative RMSE that rounding ``pre`` to ``dtype`` alone produces
    (uniform error in half an ulp either side: ulp / sqrt(12))."""

    ref = np.asarray(pre, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    if rms == 0.0:
        return 0.0
    return float(np.sqrt(np.mean(ulp(ref, dtype) ** 2) / 12.0)) / rms


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


def ulp_check(actual, pre, dtype: str, slack, ulps: float = 1.0, rmse_factor: float = 1.5) -> dict:
    """Per-element bound of the module docstring plus the relative-RMSE check.
    Returns metrics with ``ok`` and, when not ok, ``why``."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(pre, np.float64)
    if out.shape != ref.shape:
        return {"ok": False, "why": f"shape {out.shape} != {ref.shape}"}
    finite = np.isfinite(ref)
    if not np.array_equal(np.isfinite(out), finite):
        return {"ok": False, "why": "non-finite pattern differs"}
    out, ref = out[finite], ref[finite]
    slack = np.broadcast_to(np.asarray(slack, np.float64), finite.shape)[finite]
    diff = np.abs(out - ref)
    unit = ulp(np.maximum(np.abs(out), np.abs(ref)), dtype)
    bound = ulps * unit + slack + 4 * U32 * np.abs(ref)
    ratio = diff / ulp(ref, dtype)
    edges = [0.0, 0.25, 0.5, 0.75, 1.0, 1.5, 2.0, np.inf]
    metrics = error_metrics(out, ref) if out.size else {"rel_rmse": 0.0}
    rounding = rounding_rel_rmse(ref, dtype)
    metrics.update({
        "ulp_bins": edges[1:-1],
        "ulp_hist": np.histogram(ratio, bins=edges)[0].tolist() if ratio.size else [],
        "max_ulp": float(ratio.max()) if ratio.size else 0.0,
        "rounding_rel_rmse": rounding,
        "outside": int((diff > bound).sum()),
        "count": int(diff.size),
        "ok": True,
    })
    if metrics["outside"]:
        i = int(np.argmax(diff - bound))
        metrics["ok"] = False
        metrics["why"] = (f"{metrics['outside']} of {diff.size} outputs outside {ulps} ulp + "
                          f"accumulation slack; worst out={out[i]!r} pre={ref[i]!r} bound={bound[i]!r}")
    elif metrics["rel_rmse"] > rmse_factor * rounding + 1e-7:
        metrics["ok"] = False
        metrics["why"] = (f"relative RMSE {metrics['rel_rmse']:.3e} above {rmse_factor} x the "
                          f"rounding RMSE {rounding:.3e}")
    return metrics


def moe_check(actual, expected, dtype: str, ulps: float = 8.0, frac: float = 0.95,
              rel_rmse: float = 5e-3, atol: float = 2e-2, rtol: float = 1e-2,
              normwise: float = 1e-2, row_rmse: float = 3e-2, col_rmse: float = 2e-2,
              min_col_rows: int = 32) -> dict:
    """Routed-expert outputs ``[tokens, hidden]`` against the oracle's rounded
    result.

    The expert path rounds inside (gate/up to the activation dtype, the
    SwiGLU product re-quantized to e4m3 per 128-wide block), and its e4m3
    MFMAs sum in a 13-bit window, so an accumulation difference can move an
    intermediate across a rounding boundary and shift a whole token row by a
    few output ulps; no ulp-sized per-element bound holds for every element.
    Required, all of:

    * every element within the reference's own grouped-MoE tolerance,
      ``|out - ref| <= atol + rtol * |ref|`` (``assert_close(rtol=1e-2,
      atol=2e-2)``, tests/gpu/test_grouped_moe_gpu.py:130,145), and the
      normwise maximum ``max|out - ref| / max|ref| <= normwise``;
    * at least ``frac`` of the outputs within ``ulps`` ulp, and the relative
      RMSE within ``rel_rmse`` (a dropped K term of a 2048-wide gate/up or
      768-wide down reduction moves it to 2-4e-2; measured on gfx950 at the
      test shapes: 0.975-0.997 within 8 ulp, 0.6-2.2e-3);
    * the relative RMSE of every token row within ``row_rmse`` and, with at
      least ``min_col_rows`` rows, of every output column within
      ``col_rmse``: a mistake confined to one expert's rows or to a few
      columns moves too few outputs for the whole-tensor statistics, but not
      too few for its own row or column (the emulated device reaches 1.1e-2
      per row and 4e-3 per column).

    The flips move an output by the same relative amount whatever the output
    dtype, so fp16 outputs at C5's widths take ``ulps = 64`` (the relative
    width of bf16's 8; 0.85 of them lie within 8 fp16 ulps there)."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(expected, np.float64)
    if out.shape != ref.shape or out.ndim != 2:
        return {"ok": False, "why": f"shape {out.shape} against {ref.shape} (need [tokens, hidden])"}
    diff = out - ref
    ratio = np.abs(diff) / ulp(ref, dtype)
    edges = [0.0, 0.5, 1.0, 2.0, 4.0, 8.0, np.inf]
    metrics = error_metrics(out, ref)
    within = float(np.mean(ratio <= ulps))
    excess = np.abs(diff) - (atol + rtol * np.abs(ref))
    rms_row = np.sqrt(np.mean(diff * diff, axis=1)) / np.maximum(np.sqrt(np.mean(ref * ref, axis=1)), 1e-30)
    rms_col = np.sqrt(np.mean(diff * diff, axis=0)) / np.maximum(np.sqrt(np.mean(ref * ref, axis=0)), 1e-30)
    check_cols = out.shape[0] >= min_col_rows
    metrics.update({
        "ulp_bins": edges[1:-1], "ulp_hist": np.histogram(ratio, bins=edges)[0].tolist(),
        "within": within,
        "outside_tol": int((excess > 0).sum()),
        "max_tol_ratio": float((np.abs(diff) / (atol + rtol * np.abs(ref))).max()) if diff.size else 0.0,
        "max_row_rmse": float(rms_row.max()) if rms_row.size else 0.0,
        "max_col_rmse": float(rms_col.max()) if (rms_col.size and check_cols) else None,
    })
    why = []
    if metrics["outside_tol"]:
        i = np.unravel_index(int(np.argmax(excess)), excess.shape)
        why.append(f"{metrics['outside_tol']} outputs outside atol {atol} + rtol {rtol}; worst at "
                   f"{tuple(int(v) for v in i)}: out={out[i]!r} ref={ref[i]!r}")
    if metrics["normwise_max"] > normwise:
        why.append(f"normwise max {metrics['normwise_max']:.3e} above {normwise}")
    if within < frac:
        why.append(f"{within:.4f} within {ulps} ulp (need {frac})")
    if metrics["rel_rmse"] > rel_rmse:
        why.append(f"rel_rmse {metrics['rel_rmse']:.3e} above {rel_rmse}")
    if metrics["max_row_rmse"] > row_rmse:
        why.append(f"row {int(np.argmax(rms_row))} rel_rmse {metrics['max_row_rmse']:.3e} above {row_rmse}")
    if check_cols and metrics["max_col_rmse"] > col_rmse:
        why.append(f"column {int(np.argmax(rms_col))} rel_rmse {metrics['max_col_rmse']:.3e} above {col_rmse}")
    metrics["ok"] = not why
    if why:
        metrics["why"] = "; ".join(why)
    return metrics


def swiglu_check(actual, gate_pre, up_pre, dtype: str, gate_slack=0.0, up_slack=0.0,
                 rmse_factor: float = 3.0) -> dict:
    """``silu(gate) * up`` outputs against ``oracle.linear.swiglu_reference``
    of the projections' exact values.  The device's gate and up may round to
    a neighbour of the oracle's (their accumulation slack moves a value near a
    rounding boundary), so the bound propagates one ulp plus the slack of
    each input through the function: ``|silu'(g) u| (ulp(g) + gate_slack) +
    |silu(g)| (ulp(u) + up_slack)``, plus one ulp of the output and of silu's
    own rounding (times |u|); and the relative RMSE stays within
    ``rmse_factor`` x the output's rounding RMSE."""

    out = np.asarray(actual, np.float64)
    ref = np.asarray(swiglu_reference(gate_pre, up_pre, dtype), np.float64)
    gp = np.asarray(gate_pre, np.float64)
    up = np.asarray(up_pre, np.float64)
    sig = 1.0 / (1.0 + np.exp(-np.clip(gp, -80.0, 80.0)))
    silu = gp * sig
    dsilu = sig * (1.0 + gp * (1.0 - sig))
    eg = ulp(gp, dtype) + np.asarray(gate_slack, np.float64)
    eu = ulp(up, dtype) + np.asarray(up_slack, np.float64)
    slack = np.abs(dsilu * up) * eg + np.abs(silu) * eu + ulp(silu, dtype) * np.abs(up)
    return ulp_check(out, ref, dtype, slack, ulps=1.0, rmse_factor=rmse_factor)
