"""INT8 / FP8 W8A8 on gfx950 against the CPU oracle.

INT8 is bit-exact end to end (activation bytes and scales, int32 accumulators,
bf16 output).  FP8 activation bytes and scales are bit-exact; every output is
within one ulp of its dtype (plus an fp32 accumulation slack,
``gpu_helpers.assert_ulp_close``) of the exact-accumulation oracle.  Cases follow
the reference's tests/gpu/test_quant_kernels.py plus every kernel path of this
package (skinny MT=1/2/4, split-K, tiled, generic K).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import DTYPE_NAME, banner, bits, check_fp8, np32
from kairyu_amd.kernels import quant_gemm_hip as hip
from kairyu_amd.quant.fp8 import quantize_fp8
from kairyu_amd.quant.int8 import quantize_int8_weight
from kairyu_amd.quant.linear import Fp8Linear, Int8Linear
from oracle import formats, linear as olinear, numerics

pytestmark = pytest.mark.gpu


def _int8_module(k, n, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    module = Int8Linear(k, n, bias=bias)
    qw, ws = quantize_int8_weight(torch.randn(n, k, generator=g))
    module.weight.copy_(qw)
    module.weight_scale.copy_(ws)
    if bias:
        module.bias.data.normal_(generator=g)
    return module


def _fp8_module(k, n, seed=0, bias=True, per_channel=True, dynamic=True):
    g = torch.Generator().manual_seed(seed)
    module = Fp8Linear(k, n, bias=bias, activation_dynamic=dynamic)
    qw, ws = quantize_fp8(torch.randn(n, k, generator=g) * 0.02, per_channel=per_channel)
    module.weight.copy_(qw)
    if per_channel:
        module.weight_scale.copy_(ws)
    else:
        module.weight_scale = ws
    if bias:
        module.bias.data.normal_(generator=g)
    return module


# ---------------------------------------------------------------- INT8
@pytest.mark.parametrize("k", [1536, 8960])
def test_int8_activation_quantization_bit_exact(cuda, fixtures, k):
    fx = fixtures["int8_act_quant_cases"]
    banner(f"int8 act quant k={k}")
    torch.manual_seed(fx["seed"])
    x = torch.randn(fx["rows"], k, dtype=torch.bfloat16)
    x[fx["zero_row"]].zero_()
    q, s = hip._quantize_activation(x.to(cuda), torch.int8, 127.0)
    eq, es = formats.int8_quantize_rows(np32(x))
    assert np.array_equal(bits(q), eq)
    assert np.array_equal(np32(s), es)


@pytest.mark.parametrize("case", range(3))
def test_int8_fused_output_bit_exact_with_bias(cuda, fixtures, case):
    c = fixtures["int8_bitexact_cases"][case]
    banner(f"int8 bit-exact {c}")
    torch.manual_seed(c["seed"])
    module = _int8_module(c["k"], c["n"], seed=c["seed"])
    module.bias.data = module.bias.data.to(torch.bfloat16)
    x = torch.randn(c["m"], c["k"], dtype=torch.bfloat16)
    expected, _, _, _ = olinear.int8_forward(np32(x), module.weight.numpy(),
                                             module.weight_scale.numpy(), np32(module.bias))
    actual = module.to(cuda)(x.to(cuda))
    assert actual.dtype == torch.bfloat16
    assert np.array_equal(bits(actual), numerics.bf16_bits(expected).view(np.int16))


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 64, 65, 200])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_int8_accumulators_and_output_bit_exact_all_paths(cuda, m, out_dtype):
    n, k = 160, 3584  # split-K on the skinny path; beyond M = 64 the tile engine, K split 7 ways
    banner(f"int8 paths m={m} dtype={out_dtype}")
    module = _int8_module(k, n, seed=m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(100 + m)).to(out_dtype)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(),
        np32(module.bias), out_dtype=DTYPE_NAME[out_dtype])
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


# Decode path (M <= 16, K % 128 == 0, at least one 16-column tile per CU):
# N = 4104 leaves a partial last tile; K = 1536 / 4096 / 8320 selects the
# 2-, 4- and 8-wave forms (8320 = 65 stages, uneven across 8 waves); M = 8 / 9
# straddles the one- and two-instruction activation fetch.
DECODE_N = 4104


@pytest.mark.parametrize("k,m", [(1536, 1), (1536, 8), (1536, 9), (1536, 16), (4096, 8), (4096, 9), (8320, 5), (8320, 16)])
def test_int8_decode_path_bit_exact(cuda, k, m):
    banner(f"int8 decode k={k} m={m}")
    module = _int8_module(k, DECODE_N, seed=k + m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k * m)).to(torch.bfloat16)
    acc = torch.empty(m, DECODE_N, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


# Decode kernel at N = 8200 (513 column tiles, the last half used).
@pytest.mark.parametrize("k,m", [(1536, 16), (1536, 3), (4096, 9), (4096, 16)])
def test_int8_decode_wide_n_bit_exact(cuda, k, m):
    banner(f"int8 decode n=8200 k={k} m={m}")
    n = 8200
    module = _int8_module(k, n, seed=k + 3 * m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k + m)).to(torch.bfloat16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


@pytest.mark.parametrize("k,m", [(1536, 16), (4096, 5)])
def test_fp8_decode_wide_n_matches_oracle(cuda, k, m):
    banner(f"fp8 decode n=8200 k={k} m={m}")
    module = _fp8_module(k, 8200, seed=k + 3 * m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k + m)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"k={k} m={m}")


@pytest.mark.parametrize("k,m,per_channel", [(1536, 1, True), (4096, 8, False), (4096, 9, True),
                                             (8320, 16, True), (8320, 3, False)])
def test_fp8_decode_path_matches_oracle(cuda, k, m, per_channel):
    banner(f"fp8 decode k={k} m={m} per_channel={per_channel}")
    module = _fp8_module(k, DECODE_N, seed=k + m, per_channel=per_channel).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k * m)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"k={k} m={m}")


def _two_step(kind, x, module, scale_mode=0, scale_in=None):
    """Reference for the fused entries: the quantizer, then the GEMM entry."""
    cuda = x.device
    m, k = x.shape
    n = module.out_features
    stream = hip._native.stream_handle(cuda)
    xs = torch.empty(m, 1, device=cuda, dtype=torch.float32)
    out = torch.empty(m, n, device=cuda, dtype=x.dtype)
    ws = hip._workspace(cuda, int(hip._native.library().kq_w8a8_workspace_size(m, n, k)))
    wsc = module.weight_scale.float().contiguous()
    if kind == "int8":
        xq = torch.empty(m, k, device=cuda, dtype=torch.int8)
        acc = torch.empty(m, n, device=cuda, dtype=torch.int32)
        hip._native.call("kq_act_quant_i8", x.data_ptr(), hip._native.dtype_code(x.dtype), m, k, k,
                         xq.data_ptr(), xs.data_ptr(), stream)
        hip._native.call("kq_w8a8_i8_gemm", xq.data_ptr(), xs.data_ptr(), module.weight.data_ptr(),
                         wsc.data_ptr(), module.bias.data_ptr(), hip._native.dtype_code(module.bias.dtype),
                         out.data_ptr(), hip._native.dtype_code(x.dtype), acc.data_ptr(), m, n, k,
                         ws.data_ptr(), ws.numel(), stream)
        return out, acc
    xq = torch.empty(m, k, device=cuda, dtype=torch.uint8)
    hip._native.call("kq_act_quant_fp8", x.data_ptr(), hip._native.dtype_code(x.dtype), m, k, k,
                     hip._native.ptr(scale_in), scale_mode, xq.data_ptr(), xs.data_ptr(), stream)
    hip._native.call("kq_w8a8_fp8_gemm", xq.data_ptr(), xs.data_ptr(), module.weight.data_ptr(),
                     wsc.data_ptr(), int(wsc.numel() != 1), module.bias.data_ptr(),
                     hip._native.dtype_code(module.bias.dtype), out.data_ptr(),
                     hip._native.dtype_code(x.dtype), m, n, k, ws.data_ptr(), ws.numel(), stream)
    return out, None


# The fused entries: one activation row (with the decode kernel's shape
# conditions) quantizes inside the GEMM launch, more rows go through the
# quantizer and the GEMM; the bytes, the K split and the MFMA order are those
# of the quantizer + decode kernel pair either way, so outputs (bit patterns,
# NaN included) and INT8 accumulators must be identical.
@pytest.mark.parametrize("k", [1536, 4096, 8320])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_int8_fused_quant_decode_matches_two_step(cuda, k, m):
    banner(f"int8 fused decode k={k} m={m}")
    module = _int8_module(k, DECODE_N, seed=k + 7 * m).to(cuda)
    rows = _edge_rows(k, nonfinite=True)
    x = rows[[2, 3, 4, 7][:m]].to(cuda) if m <= 4 else None
    acc = torch.empty(m, DECODE_N, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x, module, accumulators=acc)
    ref, ref_acc = _two_step("int8", x, module)
    assert torch.equal(acc, ref_acc)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("k", [1536, 8320])
@pytest.mark.parametrize("m", [1, 3, 4])
@pytest.mark.parametrize("mode", ["dynamic", "static", "row"])
def test_fp8_fused_quant_decode_matches_two_step(cuda, k, m, mode):
    banner(f"fp8 fused decode k={k} m={m} {mode}")
    module = _fp8_module(k, DECODE_N, seed=k + 5 * m, dynamic=(mode != "static")).to(cuda)
    rows = _edge_rows(k, nonfinite=True)
    x = rows[[0, 2, 6, 1][:m]].to(cuda)
    scale_mode, scale_in, row_scale = 0, None, None
    if mode == "static":
        module.input_scale.fill_(0.037)
        scale_mode, scale_in = 1, module.input_scale.float().reshape(1).contiguous()
    elif mode == "row":
        row_scale = torch.tensor([0.5, 3.0e-3, 7.0, 1.0e-20][:m], device=cuda).reshape(m, 1)
        scale_mode, scale_in = 2, row_scale
    out = hip.fp8_linear_forward(x, module, activation_scale=row_scale)
    ref, _ = _two_step("fp8", x, module, scale_mode, scale_in)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


# Prefill with fewer 256x256 tiles than CUs: the tile engine splits each
# tile's K range over 2..4 work units and a reduce pass sums the raw partials
# in split order (shapes for 4 / 3 / 2 splits on 256 CUs; the second one is
# ragged in M, N (N % 8 != 0) and K).
SPLITK_SHAPES = [(1024, 2048, 4096), (1000, 2044, 4160), (1280, 4096, 3072), (1024, 8192, 2048)]


@pytest.mark.parametrize("m,n,k", SPLITK_SHAPES)
def test_int8_tile_engine_split_k_bit_exact(cuda, m, n, k):
    banner(f"int8 split-k m={m} n={n} k={k}")
    module = _int8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


# The split-K reduce writes 8 outputs per thread when N % 8 == 0 and 4 per
# thread otherwise; both forms with fp16 output and with no bias.
@pytest.mark.parametrize("m,n,k", SPLITK_SHAPES[:2])
@pytest.mark.parametrize("bias", [True, False])
def test_int8_split_k_fp16_output_bit_exact(cuda, m, n, k, bias):
    banner(f"int8 split-k fp16 m={m} n={n} k={k} bias={bias}")
    module = _int8_module(k, n, seed=m + n + 7, bias=bias).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k + 1)).to(torch.float16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    assert out.dtype == torch.float16
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(),
        np32(module.bias) if bias else None, out_dtype="float16")
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


@pytest.mark.parametrize("m,n,k", SPLITK_SHAPES[:2])
def test_fp8_split_k_fp16_output_no_bias(cuda, m, n, k):
    banner(f"fp8 split-k fp16 m={m} n={n} k={k}")
    module = _fp8_module(k, n, seed=m + n + 7, bias=False).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k + 1)).to(torch.float16)
    out = module(x.to(cuda))
    assert out.dtype == torch.float16
    check_fp8(out, x, module, label=f"fp16 m={m} n={n} k={k}", add_bias=False)


@pytest.mark.parametrize("m,n,k", SPLITK_SHAPES[:2])
def test_fp8_tile_engine_split_k_matches_oracle(cuda, m, n, k):
    banner(f"fp8 split-k m={m} n={n} k={k}")
    module = _fp8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"m={m} n={n} k={k}")


# Too few 256x256 tiles to fill half the CUs with <= 4 splits of >= 8 K blocks:
# K split up to 8 ways of >= 4 K blocks (8 ways for both shapes on 256 CUs;
# the second is ragged in N (N % 8 != 0) and K).
DEEP_SPLIT_SHAPES = [(128, 4096, 4096), (256, 2044, 4160)]


@pytest.mark.parametrize("m,n,k", DEEP_SPLIT_SHAPES)
def test_int8_deep_split_k_bit_exact(cuda, m, n, k):
    banner(f"int8 deep split-k m={m} n={n} k={k}")
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    if cus == 256:
        assert hip._native.library().kq_w8a8_workspace_size(m, n, k) == 8 * m * n * 4
    module = _int8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


@pytest.mark.parametrize("m,n,k", DEEP_SPLIT_SHAPES)
def test_fp8_deep_split_k_matches_oracle(cuda, m, n, k):
    banner(f"fp8 deep split-k m={m} n={n} k={k}")
    module = _fp8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"m={m} n={n} k={k}")


# The 128x128 tiled kernel: M > 64 with K too short to split (K = 768: six K
# blocks) and fewer 256x256 tiles than CUs; 2x2 tiles, ragged in M and N.
@pytest.mark.parametrize("m", [65, 200])
def test_w8a8_tiled_kernel_matches_oracle(cuda, m):
    banner(f"w8a8 128x128 tiles m={m}")
    n, k = 160, 768
    assert hip._native.library().kq_w8a8_workspace_size(m, n, k) == 0
    module = _int8_module(k, n, seed=m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(300 + m)).to(torch.bfloat16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)
    fmod = _fp8_module(k, n, seed=m).to(cuda)
    check_fp8(fmod(x.to(cuda)), x, fmod, label=f"128x128 fp8 m={m}")


# Whole-K tiles (at least one 256x256 tile per CU: no split-K); the second
# shape is ragged in M, N (N % 8 != 0: direct stores) and K (a 16-byte last K
# block).
WHOLE_TILE_SHAPES = [(4096, 4096, 1024), (4100, 4108, 1040)]


@pytest.mark.parametrize("m,n,k", WHOLE_TILE_SHAPES)
def test_int8_whole_tiles_bit_exact(cuda, m, n, k):
    banner(f"int8 whole tiles m={m} n={n} k={k}")
    module = _int8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
    expected, xq, xs, eacc = olinear.int8_forward(
        np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(np32(out), expected)


@pytest.mark.parametrize("m,n,k", WHOLE_TILE_SHAPES)
def test_fp8_whole_tiles_match_oracle(cuda, m, n, k):
    banner(f"fp8 whole tiles m={m} n={n} k={k}")
    module = _fp8_module(k, n, seed=m + n).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"m={m} n={n} k={k}")


def test_w8a8_workspace_size_covers_split_k(cuda):
    lib = hip._native.library()
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    # C3 prefill: 8 x 16 tiles, split in two on 256 CUs
    if cus == 256:
        assert lib.kq_w8a8_workspace_size(2048, 4096, 14336) == 2 * 2048 * 4096 * 4
    assert lib.kq_w8a8_workspace_size(8192, 4096, 14336) == 0   # a tile per CU already
    assert lib.kq_w8a8_workspace_size(16, 4096, 14336) == 0     # decode fills the CUs
    assert lib.kq_w8a8_workspace_size(0, 4096, 14336) == 0


def test_int8_generic_k_path(cuda):
    banner("int8 generic k")
    module = _int8_module(72, 24, seed=3).to(cuda)
    x = torch.randn(3, 72, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    out = module(x.to(cuda))
    expected, *_ = olinear.int8_forward(np32(x), module.weight.cpu().numpy(),
                                        module.weight_scale.cpu().numpy(), np32(module.bias))
    assert np.array_equal(np32(out), expected)


def _edge_rows(k: int, nonfinite: bool) -> torch.Tensor:
    """Rows aimed at the quantizers' corner cases: signed zeros, values far
    below the row amax, exact rounding ties of e4m3 (amax 448 -> s = 1) and of
    int8 (amax 127 -> s = 1), near-max bf16 magnitudes, and (optionally) rows
    holding +inf or NaN, which take the per-element IEEE path."""
    g = torch.Generator().manual_seed(k)
    x = torch.randn(8, k, generator=g)
    x[0, ::3] = -0.0
    x[1] = torch.randn(k, generator=g) * 1e-30
    x[1, 0] = 1.0                      # most elements quantize to (signed) zero
    ties8 = torch.tensor([1.0625, -1.1875, 0.017578125, -0.009765625, 240.0, 3.25, -6.5, 13.0])
    x[2] = ties8.repeat(k // 8 + 1)[:k]
    x[2, -1] = 448.0
    ties_i8 = torch.tensor([2.5, -3.5, 0.5, -0.5, 126.5, -1.5, 64.5, 7.0])
    x[3] = ties_i8.repeat(k // 8 + 1)[:k]
    x[3, -1] = 127.0
    x[4] = torch.randn(k, generator=g) * 1e37
    x[5, ::7] = -0.0
    if nonfinite:
        x[6, k // 2] = float("inf")
        x[7, k // 3] = float("nan")
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("k", [1536, 14336])
def test_fp8_activation_quantization_edge_values_bit_exact(cuda, k):
    banner(f"fp8 act quant edge values k={k}")
    x = _edge_rows(k, nonfinite=True)
    q, s = hip._quantize_activation(x.to(cuda), torch.float8_e4m3fn, 448.0)
    with np.errstate(invalid="ignore", divide="ignore"):
        eq, es = formats.fp8_quantize_rows(np32(x))
    assert np.array_equal(bits(q), eq)
    # scales: bit-exact where finite; any NaN where the row holds a NaN
    np.testing.assert_array_equal(np32(s), es)


@pytest.mark.parametrize("k", [1536, 3584])
def test_int8_activation_quantization_edge_values_bit_exact(cuda, k):
    banner(f"int8 act quant edge values k={k}")
    x = _edge_rows(k, nonfinite=False)
    q, s = hip._quantize_activation(x.to(cuda), torch.int8, 127.0)
    eq, es = formats.int8_quantize_rows(np32(x))
    assert np.array_equal(bits(q), eq)
    assert np.array_equal(np32(s), es)


# ----------------------------------------------------------------- FP8
@pytest.mark.parametrize("mode", ["dynamic", "static", "row"])
def test_fp8_activation_quantization_bit_exact(cuda, mode):
    banner(f"fp8 act quant {mode}")
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(6, 2304, generator=g) * 3).to(torch.bfloat16)
    x[2].zero_()
    static = torch.tensor(0.013) if mode == "static" else None
    row = (torch.rand(6, 1, generator=g) * 0.05 + 1e-3) if mode == "row" else None
    q, s = hip._quantize_activation(x.to(cuda), torch.float8_e4m3fn, 448.0,
                                    static_scale=None if static is None else static.to(cuda),
                                    row_scale=None if row is None else row.to(cuda))
    if mode == "row":
        eq = numerics.e4m3_encode(np.clip(np32(x) / row.numpy(), -448, 448))
        es = row.numpy()
    else:
        eq, es = formats.fp8_quantize_rows(np32(x), None if static is None else float(static))
    assert np.array_equal(bits(q), eq)
    assert np.array_equal(np32(s), es)


# Skinny kernel with grouped column tiles (M = 17..64 where grouping keeps
# the CUs filled): N = 4100 leaves a last group with one live column tile
# (257 tiles), K = 8192 splits K 2-4 ways; 2 (FP8 M > 32) or 4 tiles a group.
@pytest.mark.parametrize("fmt,m,k", [("int8", 17, 8192), ("int8", 40, 8192), ("int8", 64, 8192),
                                     ("fp8", 24, 8192), ("fp8", 33, 8192), ("fp8", 64, 8192),
                                     # K % step != 0: the predicated fragment loads
                                     ("int8", 40, 8208), ("fp8", 24, 8208)])
def test_grouped_skinny_matches_oracle(cuda, fmt, m, k):
    n = 4100
    banner(f"{fmt} grouped skinny m={m}")
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(5 * m)).to(torch.bfloat16)
    if fmt == "int8":
        module = _int8_module(k, n, seed=m).to(cuda)
        acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
        out = hip.int8_linear_forward(x.to(cuda), module, accumulators=acc)
        expected, xq, xs, eacc = olinear.int8_forward(
            np32(x), module.weight.cpu().numpy(), module.weight_scale.cpu().numpy(), np32(module.bias))
        assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
        assert np.array_equal(np32(out), expected)
    else:
        module = _fp8_module(k, n, seed=m).to(cuda)
        check_fp8(module(x.to(cuda)), x, module, label=f"grouped m={m}")


@pytest.mark.parametrize("m", [1, 7, 16, 24, 48, 64, 96, 300])
def test_fp8_output_matches_oracle_all_paths(cuda, m):
    n, k = 192, 14336 // 4
    banner(f"fp8 paths m={m}")
    module = _fp8_module(k, n, seed=m).to(cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    out = module(x.to(cuda))
    check_fp8(out, x, module, label=f"m={m}")


def test_fp8_per_tensor_weight_scale_and_static_input(cuda):
    banner("fp8 static")
    module = _fp8_module(64, 32, seed=2, bias=False, per_channel=False, dynamic=False)
    module.input_scale.copy_(torch.tensor(0.01))
    x = torch.randn(7, 64, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out = module.to(cuda)(x.to(cuda))
    check_fp8(out, x, module, static_scale=0.01, add_bias=False)


def test_fp8_global_per_token_scale_and_exact_amax(cuda):
    banner("fp8 global scale")
    module = _fp8_module(64, 32, seed=19)
    x = torch.randn(7, 64, generator=torch.Generator().manual_seed(19)).to(torch.bfloat16)
    amax = np32(x).__abs__().max(axis=-1, keepdims=True)
    scale = np.maximum(amax * np.float32(1.25) / np.float32(448.0), np.float32(1e-12)).astype(np.float32)
    module = module.to(cuda)
    xc = x.to(cuda)
    assert np.array_equal(np32(module.activation_amax(xc)), amax)
    out = module.forward_with_activation_scale(xc, torch.from_numpy(scale).to(cuda))
    check_fp8(out, x, module, row_scale=scale)


# ------------------------------------------------ reference ragged cases
@pytest.mark.parametrize("scheme", ["int8", "fp8"])
@pytest.mark.parametrize("shape", [(1, 64, 32), (17, 96, 40), (32, 64, 32)])
def test_ragged_shapes_match_cpu_path_without_dequantizing(cuda, fixtures, monkeypatch, scheme, shape):
    m, k, n = shape
    banner(f"ragged {scheme} {shape}")
    module = (_int8_module if scheme == "int8" else _fp8_module)(k, n, seed=0)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(0))
    cpu_out = module.forward_reference(x.to(torch.bfloat16).float())

    def forbidden(*_a, **_k):
        raise AssertionError(f"{scheme} device forward materialized its weight")

    monkeypatch.setattr(type(module), "dequantize", forbidden)
    gpu_out = module.to(cuda)(x.to(cuda, torch.bfloat16)).float().cpu()
    tol = fixtures["tolerances"][scheme]
    if scheme == "fp8":
        err = gpu_out - cpu_out
        rel = err.square().mean().sqrt() / cpu_out.square().mean().sqrt()
        assert rel.item() < tol["rel_rmse"]
        assert err.abs().max().item() < tol["max_abs_per_sqrt_k"] * k**0.5
    else:
        torch.testing.assert_close(gpu_out, cpu_out, rtol=tol["rtol"], atol=tol["atol"])


# ------------------------------------------------------------ fail closed
def test_rejects_unsupported_activation_dtype(cuda):
    module = _int8_module(64, 32).to(cuda)
    with pytest.raises(RuntimeError, match="float16/bfloat16"):
        module(torch.randn(2, 64, device=cuda))


@pytest.mark.parametrize("factory", [_int8_module, _fp8_module], ids=["int8", "fp8"])
def test_rejects_other_architectures(cuda, monkeypatch, factory):
    module = factory(64, 32).to(cuda)
    monkeypatch.setattr(hip, "_device_arch", lambda _d: "gfx942")
    with pytest.raises(RuntimeError, match="requires gfx950"):
        module(torch.randn(2, 64, device=cuda, dtype=torch.bfloat16))


def test_rejects_k_mismatch_and_misplaced_payload(cuda):
    module = _int8_module(64, 32).to(cuda)
    with pytest.raises(ValueError, match="expected K=64"):
        module(torch.randn(2, 48, device=cuda, dtype=torch.bfloat16))
    cpu_module = _int8_module(64, 32)
    with pytest.raises(RuntimeError, match="payloads"):
        hip.int8_linear_forward(torch.randn(2, 64, device=cuda, dtype=torch.bfloat16), cpu_module)


# ------------------------------------------------------------- graphs
def test_graph_replays_decode_and_split_k_paths(cuda):
    """The decode kernel (M <= 16, N = 4104) and the tile engine's split-K
    prefill (M = 1024, N = 2048: partials in the workspace, then the reduce)
    captured in one graph; every replay matches eager, with other eager work
    on the shared workspace between replays."""
    banner("w8a8 graph replay: decode + split-k")
    dec_i8 = _int8_module(4096, DECODE_N, seed=11).to(cuda)
    dec_f8 = _fp8_module(4096, DECODE_N, seed=12).to(cuda)
    sk_i8 = _int8_module(4096, 2048, seed=13).to(cuda)
    sk_f8 = _fp8_module(4096, 2048, seed=14).to(cuda)
    xd = torch.randn(16, 4096, device=cuda, dtype=torch.bfloat16)
    xp = torch.randn(1024, 4096, device=cuda, dtype=torch.bfloat16)
    mods = ((dec_i8, xd), (dec_f8, xd), (sk_i8, xp), (sk_f8, xp))
    eager = [m(x).clone() for m, x in mods]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            for m, x in mods:
                m(x)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [m(x) for m, x in mods]
    for step in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), (step, i)
        sk_f8(xp * 0.5)
        dec_i8(xd * 2.0)
        torch.cuda.synchronize()


def test_graph_replays_match_eager(cuda):
    banner("w8a8 graph replay")
    int8_mod = _int8_module(3584, 160, seed=5).to(cuda)
    fp8_mod = _fp8_module(3584, 160, seed=6).to(cuda)
    x = torch.randn(16, 3584, device=cuda, dtype=torch.bfloat16)
    eager = (int8_mod(x).clone(), fp8_mod(x).clone())
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            int8_mod(x), fp8_mod(x)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_i8 = int8_mod(x)
        out_f8 = fp8_mod(x)
    for step in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_i8, eager[0]), step
        assert torch.equal(out_f8, eager[1]), step
        # eager work between replays must not disturb the shared workspace
        int8_mod(x * 0.5)
        torch.cuda.synchronize()
