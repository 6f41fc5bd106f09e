"""Every BASELINE configuration at its exact shape, built by the same seeded
workload builders the benchmark times (``kairyu_amd.workloads``) and run
through the same ``module(x)`` call, against the CPU oracle.

* C1 AWQ N=K=4096 g128, M=16: every output.
* C2 GPTQ act-order N=28672 K=4096 g128, M in {1, 4, 16, 64, 512} (the
  decode GEMV's one-round share mode, the 64x128 and 128x256 prefill tiles):
  every column of every row for M <= 16 (every workgroup share of the decode
  GEMV), three 1024-column slices (first, middle, last) of every row above;
  the oracle's dequantization is per column, so a slice is exact.
* C3 FP8 N=4096 K=14336 with 1% x20 outliers, M in {1, 16, 2048, 8192} (decode
  kernel, 2-way split-K tile engine, whole-tile engine): every row for M <= 16,
  else 96 rows (the first and last 32 -- first and last row tile -- and 32
  seeded others) with every column; rows are independent (per-token
  quantization).
* C4 INT8 N=18944 K=3584, M in {16, 4096}: int32 accumulators and the bf16
  output bit-exact on the same row selection, and the accumulator-reporting
  call bit-identical to ``module(x)``.

W4A16 and FP8 use the per-element bound of ``gpu_helpers.assert_ulp_close``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import assert_ulp_close, banner, bits, check_fp8, check_w4a16, fp16_mfma_slack, np32
from kairyu_amd import workloads
from kairyu_amd.kernels import quant_gemm_hip as hip
from oracle import linear as olinear
from oracle.numerics import bf16_bits

pytestmark = pytest.mark.gpu


def _rows(m: int) -> np.ndarray:
    if m <= 96:
        return np.arange(m)
    middle = np.random.default_rng(m).choice(np.arange(32, m - 32), size=32, replace=False)
    return np.unique(np.concatenate([np.arange(32), middle, np.arange(m - 32, m)]))


def test_c1_awq_m16(cuda):
    banner("C1 AWQ W4A16 M=16 N=K=4096 g128")
    wl = workloads.awq_layer(m=16, device=cuda)
    out = wl.module(wl.x)
    check_w4a16(out, wl.module, wl.x.cpu(), label="C1 M=16")


@pytest.mark.parametrize("m", [1, 4, 16, 64, 512])
def test_c2_gptq_act_order(cuda, m):
    banner(f"C2 GPTQ act-order N=28672 K=4096 g128 M={m}")
    wl = workloads.gptq_layer(m=m, device=cuda)
    module = wl.module
    out = np32(module(wl.x))
    assert module._kq_gptq_operands[1][0] == hip.GIDX_PERMUTED
    x = np32(wl.x)
    qweight, qzeros = module.qweight.cpu().numpy(), module.qzeros.cpu().numpy()
    scales, g_idx = np32(module.scales), module.g_idx.cpu().numpy()
    n = module.out_features
    width = 4096 if m <= 16 else 1024
    starts = range(0, n, width) if m <= 16 else (0, n // 2 - 512, n - 1024)
    for c0 in starts:
        cols = slice(c0, c0 + width)
        pre, terms = olinear.gptq_reference(x, qweight[:, cols], qzeros[:, c0 // 8:(c0 + width) // 8],
                                            scales[:, cols], g_idx, "float16")
        assert_ulp_close(out[:, cols], pre, "float16", fp16_mfma_slack(terms, module.in_features),
                         label=f"C2 M={m} cols {c0}:{c0 + width}")


@pytest.mark.parametrize("m", [1, 16, 2048, 8192])
def test_c3_fp8(cuda, m):
    banner(f"C3 FP8 W8A8 N=4096 K=14336 M={m}")
    wl = workloads.fp8_layer(m=m, device=cuda)
    out = wl.module(wl.x)
    assert out.dtype == torch.bfloat16
    rows = torch.from_numpy(_rows(m))
    check_fp8(out.cpu()[rows], wl.x.cpu()[rows], wl.module, label=f"C3 M={m} rows {len(rows)}")


@pytest.mark.parametrize("m", [16, 4096])
def test_c4_int8_bit_exact(cuda, m):
    banner(f"C4 INT8 W8A8 N=18944 K=3584 M={m}")
    wl = workloads.int8_layer(m=m, device=cuda)
    module = wl.module
    out = module(wl.x)
    acc = torch.empty(m, module.out_features, dtype=torch.int32, device=cuda)
    out_acc = hip.int8_linear_forward(wl.x, module, accumulators=acc)
    assert torch.equal(out.view(torch.int16), out_acc.view(torch.int16))
    rows = _rows(m)
    idx = torch.from_numpy(rows).to(cuda)
    expected, _, _, eacc = olinear.int8_forward(np32(wl.x.index_select(0, idx)), module.weight.cpu().numpy(),
                                                np32(module.weight_scale), None)
    assert np.array_equal(acc.index_select(0, idx).cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(bits(out.index_select(0, idx)), bf16_bits(expected).view(np.int16))
