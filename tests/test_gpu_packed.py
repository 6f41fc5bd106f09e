"""QuantLinearPack on gfx950: one activation quantization and one GEMM launch
for several projections of the same input (the quantized counterpart of the
reference's DenseLinearPack, kairyu/models/packed_linear.py:30-218).  Every
packed output matches the CPU oracle of its own projection (INT8: bit-exact
and bit-identical to the projection run alone; FP8 / W4A16 within 1e-2
normwise and rel-RMSE), for decode and prefill row counts and under graph
replay."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import banner, check_fp8, check_w4a16, np32
from kairyu_amd.quant.fp8 import quantize_fp8
from kairyu_amd.quant.int8 import quantize_int8_weight
from kairyu_amd.quant.packed import QuantLinearPack
from kairyu_amd.quant.linear import Fp8Linear, Int8Linear
from oracle import linear as olinear
from test_gpu_w4a16 import _awq_module, _gptq_module

pytestmark = pytest.mark.gpu

SPLITS = (2048, 512, 512)   # a q / k / v style split (GQA 4:1)
K = 1024


def _int8(k, n, seed):
    g = torch.Generator().manual_seed(seed)
    m = Int8Linear(k, n, bias=True)
    qw, ws = quantize_int8_weight(torch.randn(n, k, generator=g))
    m.weight.copy_(qw)
    m.weight_scale.copy_(ws)
    m.bias.data.normal_(generator=g)
    return m


def _fp8(k, n, seed, dynamic=True, per_channel=True):
    g = torch.Generator().manual_seed(seed)
    m = Fp8Linear(k, n, bias=True, activation_dynamic=dynamic)
    qw, ws = quantize_fp8(torch.randn(n, k, generator=g) * 0.02, per_channel=per_channel)
    m.weight.copy_(qw)
    if per_channel:
        m.weight_scale.copy_(ws)
    else:
        m.weight_scale = ws
    if not dynamic:
        m.input_scale.fill_(0.02)
    m.bias.data.normal_(generator=g)
    return m


@pytest.mark.parametrize("m", [1, 16, 300])
def test_int8_pack_bit_exact(cuda, m):
    banner(f"int8 pack m={m}")
    mods = [_int8(K, n, 100 + i).to(cuda) for i, n in enumerate(SPLITS)]
    x = torch.randn(m, K, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(cuda)
    alone = [mod(x) for mod in mods]
    pack = QuantLinearPack.create(mods)
    assert pack is not None
    outs = pack(x)
    for mod, o, a in zip(mods, outs, alone):
        assert torch.equal(o, a)
        want, *_ = olinear.int8_forward(np32(x), mod.weight.cpu().numpy(), np32(mod.weight_scale),
                                        np32(mod.bias))
        assert np.array_equal(np32(o), want)


@pytest.mark.parametrize("m,dynamic,per_channel", [(1, True, True), (16, True, False), (300, True, True),
                                                   (16, False, True)])
def test_fp8_pack_matches_oracle(cuda, m, dynamic, per_channel):
    banner(f"fp8 pack m={m} dynamic={dynamic} per_channel={per_channel}")
    mods = [_fp8(K, n, 200 + i, dynamic, per_channel).to(cuda) for i, n in enumerate(SPLITS)]
    pack = QuantLinearPack.create(mods)
    assert pack is not None
    x = torch.randn(m, K, generator=torch.Generator().manual_seed(7 * m)).to(torch.bfloat16).to(cuda)
    for mod, o in zip(mods, pack(x)):
        static = None if dynamic else np32(mod.input_scale)
        check_fp8(o, x, mod, label=f"m={m}", static_scale=static)


@pytest.mark.parametrize("fmt,act_order", [("awq", False), ("gptq", False), ("gptq", True)])
@pytest.mark.parametrize("m", [1, 16, 80])
def test_w4a16_pack_matches_oracle(cuda, fmt, act_order, m):
    banner(f"w4a16 pack {fmt} act_order={act_order} m={m}")
    group = 128
    g_idx = None
    if act_order:
        g_idx = (torch.randperm(K, generator=torch.Generator().manual_seed(5)) // group).to(torch.int32)
    mods = []
    for i, n in enumerate(SPLITS):
        if fmt == "awq":
            mods.append(_awq_module(K, n, group=group, seed=300 + i, random_packed=True))
        else:
            mods.append(_gptq_module(K, n, group=group, seed=300 + i, g_idx=g_idx, random_packed=True))
    mods = [mod.to(cuda) for mod in mods]
    pack = QuantLinearPack.create(mods)
    assert pack is not None
    x = torch.randn(m, K, generator=torch.Generator().manual_seed(11 * m)).to(torch.float16)
    outs = pack(x.to(cuda))
    for mod, o in zip(mods, outs):
        check_w4a16(o, mod, x, label=f"{fmt} m={m}")


def test_pack_graph_replays_match_eager(cuda):
    banner("pack graph replay")
    group = 128
    mods = [_gptq_module(K, n, group=group, seed=400 + i, random_packed=True).to(cuda)
            for i, n in enumerate(SPLITS)]
    pack8 = QuantLinearPack.create([_fp8(K, n, 500 + i).to(cuda) for i, n in enumerate(SPLITS)])
    pack4 = QuantLinearPack.create(mods)
    x = torch.randn(4, K, generator=torch.Generator().manual_seed(3)).to(torch.float16).to(cuda)
    xb = x.to(torch.bfloat16)
    eager = [o.clone() for o in pack4(x)] + [o.clone() for o in pack8(xb)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pack4(x)
        pack8(xb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = list(pack4(x)) + list(pack8(xb))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, eager):
            assert torch.equal(a, b)
        pack4(x)  # eager work between replays
        torch.cuda.synchronize()
