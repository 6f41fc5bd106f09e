"""Pin the oracle's packed formats and quantizers, then check the package's
torch format code against it.

Pins: the reference tests' known answers (tests/golden/reference_fixtures.json),
a brute-force per-element decode written from the reference kernel's own
closed-form nibble position (quant_gemm_gpu.py:259-261 for AWQ, :377 for GPTQ),
torch.round's half-even rule, and exact-accumulation identities.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kairyu_amd.quant import awq, fp8, gptq, int8
from oracle import formats, linear as olinear, numerics


def _nibbles(word: int) -> list[int]:
    word &= 0xFFFFFFFF
    return [(word >> (4 * i)) & 0xF for i in range(8)]


# ------------------------------------------------------------ known answers
def test_awq_pack_order_known_answer(fixtures):
    fx = fixtures["awq_pack_order"]
    values = np.array([fx["values"]], dtype=np.int64)
    packed = formats.awq_pack(values)
    assert packed.shape == (1, 1)
    assert _nibbles(int(packed[0, 0])) == fx["nibbles"]
    assert np.array_equal(formats.awq_unpack(packed), values)
    ours = awq.pack_awq(torch.tensor([fx["values"]], dtype=torch.int32))
    assert _nibbles(int(ours[0, 0])) == fx["nibbles"]


def test_gptq_row_pack_known_answer(fixtures):
    fx = fixtures["gptq_row_pack"]
    values = np.array(fx["values"], dtype=np.int64).reshape(8, 1)
    packed = formats.gptq_pack_rows(values)
    assert _nibbles(int(packed[0, 0])) == fx["nibbles"]
    assert np.array_equal(formats.gptq_unpack_rows(packed), values)
    ours = gptq.pack_gptq_rows(torch.arange(8, dtype=torch.int32).reshape(8, 1))
    assert _nibbles(int(ours[0, 0])) == fx["nibbles"]


def test_gptq_zero_offset_round_trip(fixtures):
    fx = fixtures["gptq_zero_offset_roundtrip"]
    torch.manual_seed(fx["seed"])
    weight = torch.randn(*fx["shape"])
    qweight, qzeros, scales, g_idx = gptq.quantize_gptq(weight, group_size=fx["group_size"])
    restored = formats.gptq_dequantize(qweight.numpy(), qzeros.numpy(), scales.numpy(), g_idx.numpy())
    assert np.abs(restored - weight.numpy()).max() < fx["max_err"]
    # and without the +1 restore the round trip breaks: the offset is real
    q = formats.gptq_unpack_rows(qweight.numpy()).astype(np.float32)
    z_no_offset = formats.gptq_unpack_cols(qzeros.numpy()).astype(np.float32)
    g = g_idx.numpy().astype(np.int64)
    wrong = ((q - z_no_offset[g]) * scales.numpy().astype(np.float32)[g]).T
    assert np.abs(wrong - weight.numpy()).max() > fx["max_err"]


def test_fp8_clamp_before_cast(fixtures):
    fx = fixtures["fp8_clamp_before_cast"]
    w = np.array(fx["weight"], np.float32)
    q, s = formats.fp8_quantize_weight(w, per_channel=False)
    restored = formats.fp8_dequantize(q, s)
    assert not np.isnan(restored).any()
    assert np.abs(restored - w).max() / 1000.0 < fx["max_rel_err"]
    tq, ts = fp8.quantize_fp8(torch.tensor(fx["weight"]), per_channel=False)
    assert np.array_equal(tq.view(torch.uint8).numpy(), q)


@pytest.mark.parametrize("per_channel", [True, False])
def test_fp8_round_trip(fixtures, per_channel):
    fx = fixtures["fp8_roundtrip"]
    torch.manual_seed(fx["seed"])
    w = torch.randn(*fx["shape"])
    q, s = formats.fp8_quantize_weight(w.numpy(), per_channel)
    assert np.abs(formats.fp8_dequantize(q, s) - w.numpy()).max() < fx["max_abs_err"]
    tq, ts = fp8.quantize_fp8(w, per_channel=per_channel)
    assert np.array_equal(tq.view(torch.uint8).numpy(), q)
    assert np.array_equal(ts.numpy().reshape(-1), s.reshape(-1))


def test_awq_round_trip(fixtures):
    fx = fixtures["awq_roundtrip"]
    torch.manual_seed(fx["seed"])
    w = torch.randn(*fx["shape"])
    qweight, qzeros, scales = awq.quantize_awq(w, group_size=fx["group_size"])
    assert tuple(qweight.shape) == (32, 2) and tuple(qzeros.shape) == (2, 2)
    assert tuple(scales.shape) == (2, 16)
    restored = formats.awq_dequantize(qweight.numpy(), qzeros.numpy(), scales.numpy(), fx["group_size"])
    assert restored.shape == tuple(w.shape)
    assert np.abs(restored - w.numpy()).max() < fx["max_abs_err"]


# --------------------------------------------------------------- brute force
def test_awq_unpack_matches_kernel_closed_form():
    """Column n of packed word n//8 sits at bit ((n%8)//2 + (n%8)%2*4)*4."""

    rng = np.random.default_rng(5)
    words = rng.integers(-(2**31), 2**31, size=(3, 4), dtype=np.int64).astype(np.int32)
    unpacked = formats.awq_unpack(words)
    for r in range(3):
        for n in range(32):
            shift = ((n % 8) // 2 + (n % 8) % 2 * 4) * 4
            expect = (int(words[r, n // 8]) & 0xFFFFFFFF) >> shift & 0xF
            assert unpacked[r, n] == expect


def test_gptq_unpack_matches_kernel_closed_form():
    rng = np.random.default_rng(6)
    words = rng.integers(-(2**31), 2**31, size=(2, 5), dtype=np.int64).astype(np.int32)
    unpacked = formats.gptq_unpack_rows(words)
    for k in range(16):
        for n in range(5):
            expect = (int(words[k // 8, n]) & 0xFFFFFFFF) >> ((k % 8) * 4) & 0xF
            assert unpacked[k, n] == expect
    cols = formats.gptq_unpack_cols(words)
    for r in range(2):
        for n in range(40):
            assert cols[r, n] == (int(words[r, n // 8]) & 0xFFFFFFFF) >> ((n % 8) * 4) & 0xF


# ---------------------------------------------------- package vs oracle
def test_package_awq_matches_oracle_on_random_words():
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, size=(64, 48))
    z = rng.integers(0, 16, size=(4, 48))
    s = rng.uniform(0.002, 0.02, size=(4, 48)).astype(np.float16)
    qw, qz = formats.awq_pack(q), formats.awq_pack(z)
    assert np.array_equal(awq.pack_awq(torch.from_numpy(q)).numpy(), qw)
    assert np.array_equal(awq.unpack_awq(torch.from_numpy(qw)).numpy(), q)
    ours = awq.dequantize_awq(torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s), 16)
    assert np.array_equal(ours.numpy(), formats.awq_dequantize(qw, qz, s, 16))


def test_package_gptq_matches_oracle_with_act_order():
    rng = np.random.default_rng(9)
    q = rng.integers(0, 16, size=(64, 40))
    z = rng.integers(0, 16, size=(4, 40))
    s = rng.uniform(0.001, 0.01, size=(4, 40)).astype(np.float16)
    g_idx = (rng.permutation(64) // 16).astype(np.int32)
    qw, qz = formats.gptq_pack_rows(q), formats.gptq_pack_cols(z)
    assert np.array_equal(gptq.pack_gptq_rows(torch.from_numpy(q)).numpy(), qw)
    assert np.array_equal(gptq.pack_gptq_cols(torch.from_numpy(z)).numpy(), qz)
    ours = gptq.dequantize_gptq(torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s),
                                torch.from_numpy(g_idx), 16)
    assert np.array_equal(ours.numpy(), formats.gptq_dequantize(qw, qz, s, g_idx))


def test_int8_activation_quant_matches_package_bit_exact():
    torch.manual_seed(356)
    x = torch.randn(4, 1536, dtype=torch.bfloat16).float()
    x[0].zero_()
    tq, ts = int8.quantize_int8_activation(x)
    q, s = formats.int8_quantize_rows(x.numpy())
    assert np.array_equal(tq.numpy(), q)
    assert np.array_equal(ts.numpy(), s)


def test_int8_half_even_rounding_is_pinned():
    # x/s lands exactly on .5 ties: torch.round and np.rint both go to even
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5]], np.float32)
    q, s = formats.int8_quantize_rows(x)
    assert s[0, 0] == np.float32(1.0)
    assert q.tolist() == [[127, 0, 2, 2, 0, -2]]


def test_fp8_activation_quant_matches_package_bit_exact():
    torch.manual_seed(3)
    x = torch.randn(5, 320) * torch.tensor([1.0, 20.0, 1e-3, 300.0, 0.0])[:, None]
    tq, ts = fp8.quantize_fp8_activation(x)
    q, s = formats.fp8_quantize_rows(x.numpy())
    assert np.array_equal(tq.view(torch.uint8).numpy(), q)
    assert np.array_equal(ts.numpy(), s)


def test_int8_accumulation_is_exact():
    """fp64 BLAS and int64 accumulation agree exactly (reference
    test_quant_compute.py:81-92 argues the same with fp64)."""

    rng = np.random.default_rng(2)
    xq = rng.integers(-127, 128, size=(7, 3584)).astype(np.int8)
    wq = rng.integers(-127, 128, size=(33, 3584)).astype(np.int8)
    exact = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(olinear.int8_accumulate(xq, wq), exact)


def test_int8_forward_matches_package_cpu_path():
    torch.manual_seed(2)
    weight = torch.randn(8, 16)
    x = torch.randn(3, 16)
    w_q, w_s = int8.quantize_int8_weight(weight)
    ours = int8.int8_w8a8_matmul(*int8.quantize_int8_activation(x), w_q, w_s)
    out, _, _, _ = olinear.int8_forward(x.numpy(), w_q.numpy(), w_s.numpy(), out_dtype="float32")
    assert np.array_equal(ours.numpy(), out)


def test_fp8_exact_accumulation_closed_form():
    rng = np.random.default_rng(4)
    a = rng.integers(0, 256, size=(3, 512)).astype(np.uint8)
    b = rng.integers(0, 256, size=(5, 512)).astype(np.uint8)
    a[(a & 0x7F) == 0x7F] = 0  # drop NaN codes
    b[(b & 0x7F) == 0x7F] = 0
    acc = olinear.fp8_accumulate(a, b)
    # every product is a multiple of 2^-18: the sum scaled by 2^18 is an integer
    scaled = acc * 2.0**18
    assert np.array_equal(scaled, np.round(scaled))
    # and summation order does not matter
    va, vb = numerics.e4m3_decode(a).astype(np.float64), numerics.e4m3_decode(b).astype(np.float64)
    rev = (va[:, ::-1] @ vb[:, ::-1].T)
    assert np.array_equal(acc, rev)
