"""The per-element parity bound of the GPU tests (``gpu_helpers.assert_ulp_close``)
accepts an fp32-accumulating device and rejects plausible kernel mistakes.

The "device" here is the oracle itself with fp32 accumulation over 32- or
128-wide K chunks (the MFMA step widths of the W4A16 and FP8 kernels), and
the mistakes are planted in that CPU computation: a dropped K term, a wrong
group scale, an activation gathered one position off, a K block counted twice.
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import assert_ulp_close, ulp
from oracle import formats, linear as olinear
from oracle.numerics import e4m3_decode, fp16_round, to_dtype


def _fp32_chunked(a, w, chunk):
    acc = np.zeros((a.shape[0], w.shape[0]), np.float32)
    for c in range(0, a.shape[1], chunk):
        part = (a[:, c:c + chunk].astype(np.float64) @ w[:, c:c + chunk].astype(np.float64).T)
        acc = (acc + part.astype(np.float32)).astype(np.float32)
    return acc


def _gptq_case(m=4, k=4096, n=256, group=128, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(k, n))
    qweight = formats.gptq_pack_rows(q)
    qzeros = formats.gptq_pack_cols(np.full((k // group, n), 7))
    scales = rng.uniform(0.001, 0.01, size=(k // group, n)).astype(np.float16).astype(np.float32)
    g_idx = (rng.permutation(k) // group).astype(np.int32)
    x = fp16_round(rng.standard_normal((m, k)))
    return x, qweight, qzeros, scales, g_idx


def test_ulp_spacing_matches_numpy_for_fp16():
    v = np.array([1.0, 1.5, 2.0, 1000.0, 6e-5, 1e-7, 0.0, -3.0], np.float64)
    expected = np.spacing(np.abs(v).astype(np.float16)).astype(np.float64)
    assert np.array_equal(ulp(v, "float16"), expected)
    assert ulp(np.array([1.0]), "bfloat16")[0] == 2.0 ** -7
    assert ulp(np.array([3.0e-39]), "bfloat16")[0] == 2.0 ** -133


def test_w4a16_bound_accepts_fp32_accumulation_and_rejects_mistakes():
    x, qweight, qzeros, scales, g_idx = _gptq_case()
    k = x.shape[1]
    pre, terms = olinear.gptq_reference(x, qweight, qzeros, scales, g_idx, "float16")
    w = formats.w4a16_weight_fp16(formats.gptq_dequantize(qweight, qzeros, scales, g_idx))
    device = to_dtype(_fp32_chunked(x, w, 32), "float16")
    assert_ulp_close(device, pre, "float16", terms, k, label="fp32 device")

    dropped = x.copy()
    dropped[:, 1000] = 0.0
    with pytest.raises(AssertionError):
        assert_ulp_close(to_dtype(_fp32_chunked(dropped, w, 32), "float16"), pre, "float16",
                         terms, k, label="dropped k term")

    wrong_scale = scales.copy()
    wrong_scale[3] = scales[4]
    w_bad = formats.w4a16_weight_fp16(formats.gptq_dequantize(qweight, qzeros, wrong_scale, g_idx))
    with pytest.raises(AssertionError):
        assert_ulp_close(to_dtype(_fp32_chunked(x, w_bad, 32), "float16"), pre, "float16",
                         terms, k, label="wrong group scale")

    shifted = np.roll(x, 1, axis=1)
    with pytest.raises(AssertionError):
        assert_ulp_close(to_dtype(_fp32_chunked(shifted, w, 32), "float16"), pre, "float16",
                         terms, k, label="activation gathered one off")


def test_fp8_bound_accepts_fp32_accumulation_and_rejects_a_dropped_term():
    rng = np.random.default_rng(1)
    m, k, n = 4, 14336, 128
    w_bits, w_scale = formats.fp8_quantize_weight(rng.standard_normal((n, k)) * 0.02)
    x = rng.standard_normal((m, k)).astype(np.float32)
    out, x_bits, x_scale, pre = olinear.fp8_forward(x, w_bits, w_scale)
    terms = olinear.fp8_abs_terms(x_bits, w_bits, x_scale, w_scale)
    xv, wv = e4m3_decode(x_bits), e4m3_decode(w_bits)
    ws = np.asarray(w_scale, np.float32).reshape(1, -1)

    def device(xvals):
        acc = _fp32_chunked(xvals, wv, 128)
        return to_dtype(((acc * x_scale).astype(np.float32) * ws).astype(np.float32), "bfloat16")

    assert_ulp_close(device(xv), pre, "bfloat16", terms, k, label="fp32 device")
    dropped = xv.copy()
    dropped[:, 7000] = 0.0
    with pytest.raises(AssertionError):
        assert_ulp_close(device(dropped), pre, "bfloat16", terms, k, label="dropped k term")
    doubled = xv.copy()
    doubled[:, 128:256] *= 2.0
    with pytest.raises(AssertionError):
        assert_ulp_close(device(doubled), pre, "bfloat16", terms, k, label="K block twice")
