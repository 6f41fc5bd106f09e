"""The drop-in path end to end on gfx950: projections built by
``linear_factory(device="cuda")`` + ``make_linear`` (the constructor the
reference's models call) probe the device, bind the HIP forward
(``_bind_fused_forward``) and, through ``module(x)``, match the CPU oracle;
the legacy per-format modules run the same kernels."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import banner, bits, check_block_fp8, check_fp8, check_w4a16, np32
from kairyu_amd.kernels import awq_gemm_hip, fp8_gemm_hip, gptq_gemm_hip, int8_gemm_hip
from kairyu_amd.kernels import quant_gemm_hip as hip
from kairyu_amd.quant import awq as awq_format
from kairyu_amd.quant import gptq as gptq_format
from kairyu_amd.quant.block_fp8 import quantize_block_fp8
from kairyu_amd.quant.fp8 import quantize_fp8
from kairyu_amd.quant.int8 import quantize_int8_weight
from kairyu_amd.quant.linear import (
    LinearKernel,
    LinearKernelCapabilities,
    LinearRole,
    linear_factory,
    make_linear,
)
from kairyu_amd.quant.quant_config import detect_quantization
from oracle import linear as olinear

pytestmark = pytest.mark.gpu

K, N = 1024, 512

_CONFIGS = {
    "fp8": {"quant_method": "fp8", "activation_scheme": "dynamic"},
    "int8": None,
    "awq": {"quant_method": "awq", "bits": 4, "group_size": 128},
    "gptq": {"quant_method": "gptq", "bits": 4, "group_size": 128, "desc_act": True},
    "fp8_block": {"quant_method": "fp8", "weight_block_size": [128, 128]},
}
_INT8 = {"quant_method": "compressed-tensors",
         "config_groups": {"g": {"weights": {"num_bits": 8, "type": "int"},
                                 "input_activations": {"num_bits": 8, "type": "int"}}}}
_FORWARD = {"fp8": hip.fp8_linear_forward, "int8": hip.int8_linear_forward,
            "awq": hip.awq_linear_forward, "gptq": hip.gptq_linear_forward,
            "fp8_block": hip.block_fp8_linear_forward}


def test_capability_probe_on_this_device(cuda):
    caps = LinearKernelCapabilities.for_device(cuda)
    assert caps.source.startswith("rocm-gfx950;hip_lib=available"), caps.source
    for kernel in (LinearKernel.HIP_FP8_W8A8, LinearKernel.HIP_INT8_W8A8, LinearKernel.HIP_W4A16,
                   LinearKernel.HIP_FP8_BLOCK):
        assert kernel in caps.available_kernels


def _fill(module, scheme, g):
    with torch.no_grad():
        if scheme == "fp8":
            qw, ws = quantize_fp8(torch.randn(N, K, generator=g) * 0.02, per_channel=True)
            module.weight.copy_(qw)
            module.weight_scale.copy_(ws)
        elif scheme == "int8":
            qw, ws = quantize_int8_weight(torch.randn(N, K, generator=g))
            module.weight.copy_(qw)
            module.weight_scale.copy_(ws)
        elif scheme == "awq":
            groups = K // 128
            module.qweight.copy_(awq_format.pack_awq(torch.randint(0, 16, (K, N), generator=g)))
            module.qzeros.copy_(awq_format.pack_awq(torch.randint(0, 16, (groups, N), generator=g)))
            module.scales.copy_((torch.rand(groups, N, generator=g) * 0.018 + 0.002).half())
        elif scheme == "gptq":
            groups = K // 128
            module.qweight.copy_(gptq_format.pack_gptq_rows(torch.randint(0, 16, (K, N), generator=g)))
            module.qzeros.copy_(gptq_format.pack_gptq_cols(torch.full((groups, N), 7)))
            module.scales.copy_((torch.rand(groups, N, generator=g) * 0.009 + 0.001).half())
            module.g_idx.copy_((torch.randperm(K, generator=g) // 128).to(torch.int32))
        else:
            q, s = quantize_block_fp8(torch.randn(N, K, generator=g) * 0.05)
            module.weight.copy_(q)
            module.weight_scale_inv.copy_(s)


@pytest.mark.parametrize("scheme", ["fp8", "int8", "awq", "gptq", "fp8_block"])
@pytest.mark.parametrize("m", [1, 16, 100])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_factory_built_projection_runs_the_bound_hip_forward(cuda, scheme, m, dtype):
    banner(f"factory {scheme} m={m} {dtype}")
    quant = detect_quantization({"quantization_config": _CONFIGS[scheme] or _INT8})
    factory = linear_factory(quant, device=cuda, dtype=dtype)
    module = make_linear(factory, K, N, False, qualified_name="model.layers.0.mlp.down_proj",
                         role=LinearRole.MLP_DOWN, layer_index=0, shard_dim=1)
    assert module._fused_forward is _FORWARD[scheme]
    g = torch.Generator().manual_seed(m + K)
    _fill(module, scheme, g)
    module = module.to(cuda)
    x = torch.randn(m, K, generator=g).to(dtype)
    out = module(x.to(cuda))
    assert out.dtype == dtype and out.shape == (m, N)
    if scheme == "int8":
        want, *_ = olinear.int8_forward(np32(x), module.weight.cpu().numpy(), np32(module.weight_scale),
                                        None, out_dtype="bfloat16" if dtype is torch.bfloat16 else "float16")
        assert np.array_equal(np32(out), want)
    elif scheme == "fp8":
        check_fp8(out, x, module, label=f"factory fp8 m={m}")
    elif scheme == "fp8_block":
        check_block_fp8(out, x, module, label=f"factory block m={m}")
    else:
        check_w4a16(out, module, x, label=f"factory {scheme} m={m}")


@pytest.mark.parametrize("scheme,legacy", [("awq", awq_gemm_hip), ("gptq", gptq_gemm_hip),
                                           ("fp8", fp8_gemm_hip), ("int8", int8_gemm_hip)])
def test_legacy_per_format_modules_match_the_module_forward(cuda, scheme, legacy):
    quant = detect_quantization({"quantization_config": _CONFIGS[scheme] or _INT8})
    module = make_linear(linear_factory(quant, device=cuda, dtype=torch.float16), K, N, True,
                         qualified_name="model.layers.0.self_attn.o_proj",
                         role=LinearRole.ATTENTION_OUTPUT, shard_dim=1)
    _fill(module, scheme, torch.Generator().manual_seed(5))
    module = module.to(cuda)
    module.bias.data.normal_()
    x = torch.randn(4, 7, K, device=cuda, dtype=torch.float16)
    via_module = module(x)
    via_legacy = legacy.linear_forward(x, module)
    assert via_legacy.shape == (4, 7, N)
    assert np.array_equal(bits(via_module), bits(via_legacy))
