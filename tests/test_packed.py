"""Host logic of QuantLinearPack (the quantized counterpart of the reference's
DenseLinearPack, kairyu/models/packed_linear.py:30-218): which projection sets
pack, canonical buffers kept under their names, staleness detection, and the
CPU path equal to the separate projections."""

from __future__ import annotations

import pytest
import torch

from kairyu_amd.quant.fp8 import quantize_fp8
from kairyu_amd.quant.int8 import quantize_int8_weight
from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear
from kairyu_amd.quant.packed import QuantLinearPack


def _int8(k, n, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    m = Int8Linear(k, n, bias=bias)
    qw, ws = quantize_int8_weight(torch.randn(n, k, generator=g))
    m.weight.copy_(qw)
    m.weight_scale.copy_(ws)
    if bias:
        m.bias.data.normal_(generator=g)
    return m


def _fp8(k, n, seed, dynamic=True):
    g = torch.Generator().manual_seed(seed)
    m = Fp8Linear(k, n, bias=False, activation_dynamic=dynamic)
    qw, ws = quantize_fp8(torch.randn(n, k, generator=g) * 0.02, per_channel=True)
    m.weight.copy_(qw)
    m.weight_scale.copy_(ws)
    return m


def test_pack_needs_two_compatible_projections():
    a, b = _int8(64, 32, 0), _int8(64, 16, 1)
    assert QuantLinearPack.create([a]) is None
    assert QuantLinearPack.create([a, _fp8(64, 16, 2)]) is None          # mixed formats
    assert QuantLinearPack.create([a, _int8(96, 16, 3)]) is None         # different K
    assert QuantLinearPack.create([a, _int8(64, 16, 4, bias=False)]) is None  # mixed bias
    hooked = _int8(64, 16, 5)
    hooked.register_forward_hook(lambda *args: None)
    assert QuantLinearPack.create([a, hooked]) is None
    assert QuantLinearPack.create([_fp8(64, 16, 6), _fp8(64, 16, 7, dynamic=False)]) is None
    s1, s2 = _fp8(64, 16, 8, dynamic=False), _fp8(64, 16, 9, dynamic=False)
    s2.input_scale.fill_(2.0)
    assert QuantLinearPack.create([s1, s2]) is None                    # different static scales
    assert QuantLinearPack.create([a, b]) is not None


def test_w4a16_pack_rules():
    a, b = AwqLinear(128, 32, bias=False, group_size=32), AwqLinear(128, 48, bias=False, group_size=32)
    assert QuantLinearPack.create([a, b]) is not None
    assert QuantLinearPack.create([a, AwqLinear(128, 32, bias=False, group_size=64)]) is None
    assert QuantLinearPack.create([a, AwqLinear(128, 40, bias=False, group_size=32)]) is None  # N % 16
    g1, g2 = GptqLinear(128, 32, bias=False, group_size=32), GptqLinear(128, 32, bias=False, group_size=32)
    g1.g_idx.copy_((torch.arange(128) // 32).to(torch.int32))
    g2.g_idx.copy_(torch.flip(g1.g_idx, [0]))
    assert QuantLinearPack.create([g1, g2]) is None                    # different g_idx
    g2.g_idx.copy_(g1.g_idx)
    assert QuantLinearPack.create([g1, g2]) is not None


def test_w8a8_pack_keeps_canonical_buffers_as_views():
    mods = [_int8(64, 32, 10), _int8(64, 16, 11), _int8(64, 16, 12)]
    before = [dict(m.state_dict()) for m in mods]
    before = [{k: v.clone() for k, v in sd.items()} for sd in before]
    pack = QuantLinearPack.create(mods)
    assert pack.out_features == (32, 16, 16)
    storage = mods[0].weight.untyped_storage().data_ptr()
    for m, sd in zip(mods, before):
        assert m.weight.untyped_storage().data_ptr() == storage
        assert set(m.state_dict()) == set(sd)
        for key, value in sd.items():
            assert torch.equal(m.state_dict()[key], value), key
    assert pack.is_current() and pack.matches(mods)
    # an in-place update through a canonical view is seen by the pack
    mods[1].weight.fill_(3)
    assert torch.equal(pack._weight[32:48], torch.full((16, 64), 3, dtype=torch.int8))
    # replacing a canonical buffer detaches it from the pack
    mods[2].weight = mods[2].weight.clone()
    assert not pack.is_current()
    with pytest.raises(RuntimeError, match="no longer match"):
        pack(torch.randn(2, 64))


def test_cpu_call_equals_separate_projections():
    mods = [_int8(64, 32, 20), _int8(64, 16, 21)]
    pack = QuantLinearPack.create(mods)
    x = torch.randn(3, 5, 64)
    outs = pack(x)
    assert [tuple(o.shape) for o in outs] == [(3, 5, 32), (3, 5, 16)]
    for o, m in zip(outs, mods):
        assert torch.equal(o, m(x))


def test_gptq_pack_rebuild_rejects_a_diverged_g_idx():
    """The pack gathers x once through the first projection's permutation, so
    a g_idx updated in place on one projection must stop the pack at its next
    operand rebuild instead of producing silently wrong rows."""
    perm = (torch.randperm(128, generator=torch.Generator().manual_seed(3)) // 32).to(torch.int32)
    g1, g2 = GptqLinear(128, 32, bias=False, group_size=32), GptqLinear(128, 32, bias=False, group_size=32)
    g1.g_idx.copy_(perm)
    g2.g_idx.copy_(perm)
    pack = QuantLinearPack.create([g1, g2])
    assert pack is not None
    g2.g_idx.copy_(torch.flip(perm, [0]))
    with pytest.raises(RuntimeError, match="one g_idx"):
        pack._operands(torch.device("cpu"))
