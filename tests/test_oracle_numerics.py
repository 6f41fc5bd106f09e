"""Pin the oracle's bit-level numerics against torch's own CPU casts.

torch is the library routine the reference's CPU path calls for these casts
(kairyu/quant/fp8.py:29,44 ``.to(torch.float8_e4m3fn)``; bf16 model dtype), so
agreement here pins the numpy restatement.  A wrong rounding rule, exponent
bias or subnormal quantum fails one of these.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import numerics


def _torch_e4m3_bits(values: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(values.astype(np.float32)).to(torch.float8_e4m3fn)
    return t.view(torch.uint8).numpy()


def test_e4m3_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = numerics.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])


def test_e4m3_encode_matches_torch_on_representables_and_midpoints():
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    vals = np.unique(vals[np.isfinite(vals)])
    mids = (vals[:-1].astype(np.float64) + vals[1:]) / 2.0
    probes = np.concatenate([
        vals,
        mids.astype(np.float32),
        np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
        np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
    ]).astype(np.float32)
    probes = probes[np.abs(probes) <= 448.0]
    assert np.array_equal(numerics.e4m3_encode(probes), _torch_e4m3_bits(probes))


def test_e4m3_encode_matches_torch_on_random_values():
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(1_000_000) * np.exp2(rng.integers(-14, 9, 1_000_000))).astype(np.float32)
    v = np.clip(v, -448.0, 448.0)
    assert np.array_equal(numerics.e4m3_encode(v), _torch_e4m3_bits(v))


def test_e4m3_encode_subnormals_and_signed_zero():
    v = np.array([0.0, -0.0, 2.0**-9, 2.0**-10, 3 * 2.0**-10, 2.0**-6 - 2.0**-10, -2.0**-7],
                 dtype=np.float32)
    assert np.array_equal(numerics.e4m3_encode(v), _torch_e4m3_bits(v))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(1_000_000) * np.exp2(rng.integers(-60, 60, 1_000_000))).astype(np.float32)
    # exact ties: low 16 bits == 0x8000, with both parities of bit 16
    base = v[:4096].view(np.uint32) & np.uint32(0xFFFE0000)
    ties = np.concatenate([base | 0x8000, base | 0x18000]).astype(np.uint32).view(np.float32)
    v = np.concatenate([v, ties, np.array([np.inf, -np.inf, 0.0, -0.0, np.nan], np.float32)])
    ours = numerics.bf16_round(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_w4a16_activation_saturates_only_finite_bf16():
    x = np.array([70000.0, -70000.0, 65504.0, np.inf, -np.inf, 1.5], np.float32)
    out = numerics.w4a16_activation(x, "bfloat16")
    assert out[0] == 65504.0 and out[1] == -65504.0 and out[2] == 65504.0
    assert np.isposinf(out[3]) and np.isneginf(out[4]) and out[5] == 1.5
    # fp16 activations are not saturated (they cannot exceed the range)
    assert np.isinf(numerics.w4a16_activation(np.array([1e6], np.float32), "float16")[0])
