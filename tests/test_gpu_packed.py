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


# ---------------------------------------------------------------- SwiGLU
# silu(gate(x)) * up(x) of a (gate, up) pack (kairyu/models/layers.py:243-244).
# W4A16: one kq_w4a16_tiled_swiglu_gemm call; decode shapes apply SwiGLU in
# the GEMV epilogue (K <= 4096) or in the reduce of its K chunks (K > 4096),
# prefill shapes (M > 64) in the prefill epilogue, others run the tiled GEMM
# and the elementwise pass.  W8A8: one kq_w8a8_*_swiglu_linear call; prefill
# shapes apply SwiGLU in the tile engine's epilogue, M <= 64 in the decode
# or skinny GEMM's (or their split-K reduce), others run the packed GEMM and
# kq_swiglu.
_SWIGLU_CASES = [
    # (scheme, m, k, width, dtype, bias)
    ("gptq", 1, 4096, 4096, torch.float16, False),
    ("gptq", 16, 4096, 4096, torch.bfloat16, True),
    ("gptq-ao", 4, 4096, 4096, torch.float16, False),
    ("gptq-sym", 16, 4096, 4096, torch.float16, False),
    ("gptq-sym-ao", 1, 4096, 4096, torch.bfloat16, False),
    ("awq", 5, 4096, 4096, torch.float16, True),
    ("gptq", 100, 1024, 1024, torch.bfloat16, False),      # prefill, 64 x 256 SwiGLU tiles
    ("gptq-ao", 200, 1024, 14336, torch.float16, True),     # prefill, 128 x 256 SwiGLU tiles
    ("gptq-sym-ao", 7, 4128, 512, torch.float16, False),   # skinny shape: two passes
    ("awq", 64, 2048, 1024, torch.float16, False),
    # W4A16 prefill SwiGLU epilogue: a ragged last 256-column tile, act-order, real widths
    ("gptq-ao", 48, 2048, 1040, torch.float16, True),
    ("awq", 300, 4096, 11008, torch.bfloat16, False),      # 128 x 512 SwiGLU tiles (two pairs per wave)
    ("gptq-ao", 512, 1024, 10880, torch.float16, True),     # ... ending in a half-used 512-column tile
    # real MLP widths: 2-4 gate/up pairs per workgroup, uneven shares, K = 2048 (S = 4)
    ("gptq-sym-ao", 1, 4096, 14336, torch.float16, False),
    ("gptq", 16, 4096, 14336, torch.bfloat16, False),
    ("gptq-sym", 1, 4096, 11008, torch.float16, False),
    ("awq", 16, 4096, 11008, torch.float16, False),
    ("gptq-sym-ao", 16, 2048, 14336, torch.float16, False),
    ("gptq", 1, 2048, 11008, torch.bfloat16, True),
    # decode, K past one GEMV pass: the K chunks' reduce applies SwiGLU
    ("gptq-ao", 1, 8192, 2048, torch.float16, False),
    ("gptq", 16, 5120, 1024, torch.bfloat16, True),
    ("awq", 4, 14336, 1024, torch.float16, False),
    ("gptq-sym-ao", 16, 4224, 512, torch.float16, False),   # K % 256 == 128: three chunks
    ("fp8", 1, 2048, 2048, torch.bfloat16, True),
    ("fp8", 300, 1024, 1024, torch.float16, False),
    # decode shapes: SwiGLU in the decode GEMM's epilogue (8 gate + 8 up rows
    # per workgroup), one-row fused quantization at M = 1
    ("fp8", 16, 4096, 14336, torch.bfloat16, True),
    ("fp8-static", 1, 4096, 1004, torch.float16, True),
    ("int8", 1, 3584, 9472, torch.bfloat16, False),
    ("int8", 9, 4096, 1028, torch.float16, True),
    # M = 17-64 (skinny kernel): one K range per tile, and split K whose
    # reduce pairs the columns
    ("fp8", 32, 4096, 14336, torch.bfloat16, True),
    ("fp8", 40, 4096, 2048, torch.float16, False),
    ("int8", 33, 8192, 512, torch.bfloat16, False),
    # prefill shapes: SwiGLU in the tile engine's epilogue (>= 128 tiles of 256 x 256)
    ("fp8", 1024, 1024, 4096, torch.bfloat16, True),
    ("int8", 2048, 1024, 2048, torch.float16, False),
    ("int8", 16, 2048, 1024, torch.bfloat16, True),
]


def _swiglu_pair(scheme, k, width, bias, seed):
    gen = torch.Generator().manual_seed(seed)
    if scheme in ("fp8", "fp8-static", "int8"):
        make = {"fp8": _fp8, "int8": _int8, "fp8-static": lambda k, n, s: _fp8(k, n, s, dynamic=False)}[scheme]
        mods = [make(k, width, seed + i) for i in range(2)]
        if not bias:
            for m in mods:
                m.bias = None
        return mods
    group = 128
    mods = []
    for i in range(2):
        if scheme == "awq":
            mods.append(_awq_module(k, width, group=group, seed=seed + i, bias=bias, random_packed=True))
            continue
        g_idx = None
        if scheme.endswith("-ao"):
            g_idx = (torch.randperm(k, generator=torch.Generator().manual_seed(seed)) // group).to(torch.int32)
        m = _gptq_module(k, width, group=group, seed=seed + i, bias=bias, g_idx=g_idx, random_packed=True)
        if g_idx is not None:
            m.g_idx.copy_(g_idx)
        if "-sym" in scheme:
            from kairyu_amd.quant import gptq as gptq_format
            m.qzeros.copy_(gptq_format.pack_gptq_cols(torch.full((m.qzeros.shape[0], width), 7)))
        mods.append(m)
    return mods


@pytest.mark.parametrize("case", _SWIGLU_CASES, ids=lambda c: "-".join(map(str, c[:4])) + ("-b" if c[5] else ""))
def test_swiglu_pack_matches_oracle(cuda, case):
    from gpu_helpers import check_swiglu

    scheme, m, k, width, dtype, bias = case
    banner(f"swiglu pack {case}")
    gate, up = (mod.to(cuda) for mod in _swiglu_pair(scheme, k, width, bias, seed=31 * m + k))
    pack = QuantLinearPack.create([gate, up])
    assert pack is not None
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + k)).to(dtype)
    out = pack.swiglu(x.to(cuda))
    assert out.shape == (m, width) and out.dtype == dtype
    check_swiglu(out, gate, up, x, label=str(case))
    # the same call again (derived operands cached) gives the same bits
    assert torch.equal(pack.swiglu(x.to(cuda)), out)


def test_swiglu_pack_in_a_graph(cuda):
    """Decode GEMV with the SwiGLU epilogue captured once and replayed."""

    gate, up = (mod.to(cuda) for mod in _swiglu_pair("gptq-sym-ao", 4096, 4096, False, seed=5))
    pack = QuantLinearPack.create([gate, up])
    x = torch.randn(16, 4096, generator=torch.Generator().manual_seed(6)).to(torch.float16).to(cuda)
    eager = pack.swiglu(x).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pack.swiglu(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pack.swiglu(x)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("scheme,m,k,width", [("fp8", 16, 4096, 4096), ("fp8", 40, 14336, 1024),
                                               ("int8", 24, 3584, 2048)])
def test_w8a8_swiglu_pack_in_a_graph(cuda, scheme, m, k, width):
    """W8A8 decode / skinny GEMMs with the SwiGLU epilogue (and, at K = 14336,
    the split-K reduce that pairs the columns) captured once, replayed with
    eager work between the replays, every replay equal to the eager call."""

    gate, up = (mod.to(cuda) for mod in _swiglu_pair(scheme, k, width, True, seed=m + k))
    pack = QuantLinearPack.create([gate, up])
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(cuda)
    eager = pack.swiglu(x).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pack.swiglu(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pack.swiglu(x)
    other = torch.randn(m, k, generator=torch.Generator().manual_seed(m + 1)).to(torch.bfloat16).to(cuda)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        pack.swiglu(other)  # eager work between replays reuses the workspace
        torch.cuda.synchronize()


@pytest.mark.parametrize("scheme", ["gptq-ao", "awq"])
def test_swiglu_pack_holds_the_only_tiled_copy(cuda, scheme):
    """After ``pack.swiglu`` neither projection keeps a tiled operand of its
    own: the interleaved (gate, up) operand is the only derived copy of the
    4-bit weights (a second per-module copy would add half of gate/up's
    weight bytes per layer)."""

    gate, up = (mod.to(cuda) for mod in _swiglu_pair(scheme, 2048, 2048, False, seed=8))
    pack = QuantLinearPack.create([gate, up])
    assert pack is not None
    for mod in (gate, up):
        assert "_kq_gptq_operands" not in mod.__dict__ and "_kq_awq_operands" not in mod.__dict__
    x = torch.randn(4, 2048, generator=torch.Generator().manual_seed(9)).to(torch.float16).to(cuda)
    pack.swiglu(x)
    for mod in (gate, up):
        assert "_kq_gptq_operands" not in mod.__dict__ and "_kq_awq_operands" not in mod.__dict__


def test_swiglu_pack_rejects_diverged_g_idx(cuda):
    """An act-order pack whose up projection's ``g_idx`` is changed in place to
    another permutation cannot share one activation gather: the rebuilt
    operand raises instead of applying gate's permutation to up."""

    gate, up = (mod.to(cuda) for mod in _swiglu_pair("gptq-ao", 2048, 2048, False, seed=10))
    pack = QuantLinearPack.create([gate, up])
    x = torch.randn(4, 2048, generator=torch.Generator().manual_seed(11)).to(torch.float16).to(cuda)
    pack.swiglu(x)
    other = (torch.randperm(2048, generator=torch.Generator().manual_seed(12)) // 128).to(torch.int32)
    up.g_idx.copy_(other.to(cuda))
    with pytest.raises(RuntimeError, match="one g_idx"):
        pack.swiglu(x)


@pytest.mark.parametrize("scheme,m,k,width,dtype,bias", [
    ("fp8", 1024, 1024, 4096, torch.bfloat16, True),
    ("int8", 2048, 1024, 2048, torch.float16, False),
    # decode GEMM epilogue, every decode form: 4 waves (K = 4096, >= 1 tile
    # per CU), 16 waves (K = 4096, few tiles), 8 waves (K = 14336), 2 waves
    # (K = 2048 / 3584); fused quantization at M = 1; ragged widths
    ("fp8", 1, 4096, 4096, torch.bfloat16, True),
    ("fp8", 2, 4096, 1004, torch.float16, False),
    ("fp8", 16, 14336, 2048, torch.bfloat16, True),
    ("fp8-static", 16, 4096, 14336, torch.float16, False),
    ("fp8-static", 1, 2048, 2052, torch.bfloat16, True),
    ("int8", 1, 2048, 2048, torch.float16, True),
    ("int8", 16, 3584, 9472, torch.bfloat16, False),
    ("int8", 9, 4096, 1028, torch.float16, True),
    ("int8", 4, 14336, 4096, torch.bfloat16, True),
    # skinny kernel (M = 17-64, or K % 128 != 0): one K range per tile,
    # 2- and 4-way split K (reduce with SwiGLU), ragged K steps
    ("fp8", 32, 4096, 14336, torch.bfloat16, True),
    ("fp8", 64, 4096, 14336, torch.bfloat16, False),
    ("fp8", 48, 14336, 1024, torch.float16, True),
    ("fp8", 32, 14336, 1024, torch.float16, True),
    ("fp8", 16, 4112, 2048, torch.bfloat16, False),
    ("fp8-static", 24, 4096, 1000, torch.float16, True),
    ("int8", 64, 14336, 1024, torch.float16, True),
    ("int8", 24, 2048, 1000, torch.bfloat16, True),
    ("int8", 33, 8192, 512, torch.float16, False),
    ("int8", 50, 1040, 520, torch.float16, True),
    ("int8", 40, 8208, 1024, torch.bfloat16, True),   # grouped tiles, K % 64 != 0, 8-way split
])
def test_w8a8_swiglu_epilogue_bit_identical_to_two_passes(cuda, scheme, m, k, width, dtype, bias):
    """The SwiGLU epilogues (tile engine for prefill shapes, decode and
    skinny GEMMs and their split-K reduce for M <= 64) give the bits of the
    packed GEMM followed by the elementwise pass (kq_swiglu) on the same
    call."""
    from kairyu_amd import _native

    gate, up = (mod.to(cuda) for mod in _swiglu_pair(scheme, k, width, bias, seed=m + width))
    pack = QuantLinearPack.create([gate, up])
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(width)).to(dtype).to(cuda)
    fused = pack.swiglu(x)
    both = pack(x)
    packed = torch.cat(both, dim=-1).contiguous()
    two = torch.empty(m, width, device=cuda, dtype=dtype)
    _native.call("kq_swiglu", packed.data_ptr(), packed.stride(0), 0, _native.dtype_code(dtype), two.data_ptr(),
                 m, width, _native.stream_handle(torch.device(cuda)))
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
