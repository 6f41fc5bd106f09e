"""A decode step of quantized linears (GPTQ act-order W4A16 -> FP8 W8A8)
captured once per batch bucket: replays equal the eager step on the same
padded input bit for bit, the real rows match the CPU oracle, eager work
between replays does not disturb them, oversize batches run eagerly and an
invalidated set re-captures against updated weights."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import banner, check_fp8, check_w4a16
from kairyu_amd.graphs import BucketedGraphs
from test_gpu_packed import _fp8
from test_gpu_w4a16 import _gptq_module

pytestmark = pytest.mark.gpu

K, H = 1024, 2048


def _step_modules(cuda):
    g_idx = (torch.randperm(K, generator=torch.Generator().manual_seed(9)) // 128).to(torch.int32)
    up = _gptq_module(K, H, group=128, seed=21, g_idx=g_idx, random_packed=True).to(cuda)
    down = _fp8(H, K, 22).to(cuda)
    return up, down


def test_bucketed_decode_graphs(cuda):
    banner("bucketed decode graphs")
    up, down = _step_modules(cuda)

    def step(x):
        return down(up(x))

    graphs = BucketedGraphs(step, K, 16, dtype=torch.float16, device=cuda)
    graphs.capture_all()
    assert graphs.buckets == (1, 2, 4, 8, 16)
    gen = torch.Generator().manual_seed(5)
    for rows in (1, 3, 5, 16, 3):
        x = torch.randn(rows, K, generator=gen).to(torch.float16).to(cuda)
        got = graphs.run(x).clone()
        bucket = next(b for b in graphs.buckets if b >= rows)
        padded = torch.zeros(bucket, K, dtype=torch.float16, device=cuda)
        padded[:rows] = x
        assert torch.equal(got, step(padded)[:rows])   # eager work between replays too
        hidden = up(x)
        check_w4a16(hidden, up, x.cpu(), label=f"up rows={rows}")
        check_fp8(got, hidden, down, label=f"step rows={rows}")
    big = torch.randn(20, K, generator=gen).to(torch.float16).to(cuda)
    assert torch.equal(graphs.run(big), step(big))     # beyond the largest bucket: eager

    # weights swapped in place: the captured graphs are stale until re-captured
    with torch.no_grad():
        down.weight.copy_(torch.flip(down.weight, [0]))
    graphs.invalidate()
    graphs.capture_all()
    x = torch.randn(4, K, generator=gen).to(torch.float16).to(cuda)
    assert torch.equal(graphs.run(x), step(x))
    graphs.close()
