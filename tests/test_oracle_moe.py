"""CPU checks of the MoE oracle (routing, block-FP8 GEMM, combine) and of the
package's CPU routing / mixing against it.

Pins: the reference's router and combine fixtures
(tests/unit/test_moe_precision.py:97-154,194-248, transcribed into
tests/golden/reference_fixtures.json); the block GEMM against
dequantize-then-matmul (a different formula for the same quantity) and a
brute-force loop.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kairyu_amd import moe as hmoe
from oracle import formats, moe
from oracle.numerics import bf16_round, e4m3_decode


def test_router_fixtures(fixtures):
    for name in ("router_fixed", "router_ties"):
        fx = fixtures[name]
        idx, w = moe.route_topk(np.array([fx["logits"]], np.float32), fx["top_k"])
        assert idx[0].tolist() == fx["expected_indices"], name
        assert abs(float(w.sum()) - 1.0) < 1e-6


@pytest.mark.parametrize("norm", [True, False])
def test_router_weights_are_the_softmax_of_the_selection(norm):
    rng = np.random.default_rng(5)
    logits = bf16_round(rng.standard_normal((50, 60)).astype(np.float32))
    idx, w = moe.route_topk(logits, 6, norm)
    for t in range(50):
        assert list(idx[t]) == sorted(range(60), key=lambda e: (-logits[t, e], e))[:6]
        src = logits[t, idx[t]] if norm else logits[t]
        p = np.exp(src.astype(np.float64) - src.max())
        p /= p.sum()
        expect = p if norm else p[idx[t]]
        np.testing.assert_allclose(w[t], expect, rtol=2e-6, atol=0)


def test_combine_fixtures(fixtures):
    fx = fixtures["combine_fp32_before_cast"]
    y = np.array(fx["expert_values"], np.float32).reshape(1, 2, 1)
    w = np.array([fx["weights"]], np.float32)
    got = bf16_round(moe.combine(y, w))[0, 0]
    expected = bf16_round(np.float32(y[0, 0, 0] * w[0, 0]) + np.float32(y[0, 1, 0] * w[0, 1]))
    premature = bf16_round(bf16_round(y[0, 0, 0] * bf16_round(w[0, 0]))
                           + bf16_round(y[0, 1, 0] * bf16_round(w[0, 1])))
    assert got == expected and got != premature

    fx = fixtures["combine_slot_order"]
    y = np.array(fx["expert_values"], np.float32).reshape(1, 4, 1)
    w = np.array([fx["weights"]], np.float32)
    got = bf16_round(moe.combine(y, w))[0, 0]
    owners = fx["ep2_owner_slots"]
    per_owner = sum(
        float(bf16_round(np.float32(sum(np.float64(y[0, s, 0]) * w[0, s] for s in slots))).item())
        for slots in owners
    )
    assert got != bf16_round(np.float32(per_owner))
    ref = np.float32(0)
    for s in range(4):
        ref = np.float32(ref + np.float32(y[0, s, 0] * w[0, s]))
    assert got == bf16_round(ref)


def test_block_gemm_equals_dequantized_matmul_and_brute_force():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 384)).astype(np.float32)
    w = (rng.standard_normal((256, 384)) * 0.05).astype(np.float32)  # N/128 != K/128
    xq, xs = formats.block_fp8_quantize_rows(x)
    wq, ws = formats.block_fp8_quantize_weight(w)
    got = moe.block_gemm(xq, xs, wq, ws)
    xdq = e4m3_decode(xq).astype(np.float64) * np.repeat(xs.astype(np.float64), 128, axis=1)
    wdq = e4m3_decode(wq).astype(np.float64) * np.repeat(np.repeat(ws.astype(np.float64), 128, 0), 128, 1)
    np.testing.assert_allclose(got, xdq @ wdq.T, rtol=1e-12, atol=1e-12)
    # the float32 dequantization of the formats module agrees to fp32 rounding
    np.testing.assert_allclose(formats.block_fp8_dequantize(wq, ws), wdq, rtol=2**-23, atol=0)
    xv, wv = e4m3_decode(xq), e4m3_decode(wq)
    for r, n in ((0, 0), (4, 255), (2, 130)):
        ref = sum(float(xv[r, k]) * float(wv[n, k]) * float(xs[r, k // 128]) * float(ws[n // 128, k // 128])
                  for k in range(384))
        assert abs(got[r, n] - ref) <= 1e-9 * max(1.0, abs(ref))


def test_host_cpu_routing_matches_oracle():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(33, 24, generator=g).to(torch.bfloat16)
    logits[:, 5] = logits[:, 6]  # ties
    for norm in (True, False):
        idx, w = hmoe.route_logits(logits, 4, norm)
        oidx, ow = moe.route_topk(logits.float().numpy(), 4, norm)
        assert idx.dtype == torch.int64 and w.dtype == torch.float32
        assert np.array_equal(idx.numpy(), oidx)
        np.testing.assert_allclose(w.numpy(), ow, rtol=2e-6, atol=0)


def test_cpu_block_matches_oracle():
    torch.manual_seed(11)
    block = hmoe.Qwen3BlockFp8MoeBlock(256, 128, 8, 2)
    hmoe.quantize_experts(block, torch.randn(8, 256, 256) * 0.05, torch.randn(8, 256, 128) * 0.05)
    with torch.no_grad():
        block.gate.weight.normal_(0, 0.1)
    block.gate.to(torch.bfloat16)
    x = torch.randn(19, 256).to(torch.bfloat16)
    with torch.no_grad():
        out = block(x)
        logits = block.gate(x)
    idx, w = moe.route_topk(logits.float().numpy(), 2)
    w13 = np.stack([np.concatenate([e.gate_proj.weight.view(torch.uint8).numpy(),
                                    e.up_proj.weight.view(torch.uint8).numpy()]) for e in block.experts])
    s13 = np.stack([np.concatenate([e.gate_proj.weight_scale_inv.numpy(),
                                    e.up_proj.weight_scale_inv.numpy()]) for e in block.experts])
    w2 = np.stack([e.down_proj.weight.view(torch.uint8).numpy() for e in block.experts])
    s2 = np.stack([e.down_proj.weight_scale_inv.numpy() for e in block.experts])
    expected = moe.moe_forward(x.float().numpy(), idx, w, w13, s13, w2, s2)
    err = np.abs(out.float().numpy() - expected).max() / np.abs(expected).max()
    assert err < 1e-2
