"""Every advertised quant scheme generates through a whole model on gfx950.

Counterpart of the reference's ``tests/gpu/test_quant_full_model_gpu.py:62-77``:
a tiny Llama (the reference's ``TINY`` config, ``tests/quant_checkpoint_fixtures.py:11-19``,
seed 41) has every q/k/v/o and gate/up/down projection quantized by this
package's quantizers (group size 16 for AWQ / GPTQ, per-channel FP8 / INT8, as
the reference fixtures do) and built through ``linear_factory`` +
``make_linear`` from the scheme's ``quantization_config``.  Greedy decoding of
8 tokens after ``range(10)`` runs once on the CPU in fp32 (the modules'
reference forwards) and once on the GPU with the projections in bf16 through
the HIP kernels; the two must agree on at least half of the tokens and the GPU
output must not be degenerate.

The rest of the model (embeddings, RMSNorm, rotary attention) is the
transformers implementation and stays in fp32 on the GPU: attention is not
part of this package, and torch's batched bf16 products are kept out of the
run.  NVFP4 (an NVIDIA-only format) is not supported on gfx950 and is not
listed.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

TINY = dict(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
            intermediate_size=128, vocab_size=256, max_position_embeddings=512)

QUANT_CONFIGS = {
    "fp8": {"quant_method": "compressed-tensors",
            "config_groups": {"group_0": {
                "weights": {"type": "float", "num_bits": 8, "strategy": "channel"},
                "input_activations": {"type": "float", "num_bits": 8, "dynamic": True}}},
            "ignore": ["lm_head"]},
    "int8": {"quant_method": "compressed-tensors",
             "config_groups": {"group_0": {
                 "weights": {"type": "int", "num_bits": 8, "strategy": "channel"},
                 "input_activations": {"type": "int", "num_bits": 8, "dynamic": True}}},
             "ignore": ["lm_head"]},
    "awq": {"quant_method": "awq", "bits": 4, "group_size": 16, "version": "gemm", "zero_point": True},
    "gptq": {"quant_method": "gptq", "bits": 4, "group_size": 16, "desc_act": False, "sym": True},
}

_ROLES = {"q_proj": "ATTENTION_QUERY", "k_proj": "ATTENTION_KEY", "v_proj": "ATTENTION_VALUE",
          "o_proj": "ATTENTION_OUTPUT", "gate_proj": "MLP_GATE", "up_proj": "MLP_UP",
          "down_proj": "MLP_DOWN"}


class _Bf16Projection(nn.Module):
    """Runs a quantized projection on bf16 activations inside an fp32 model."""

    def __init__(self, inner: nn.Module) -> None:
        super().__init__()
        self.inner = inner

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.inner(x.to(torch.bfloat16)).to(x.dtype)


def _quantized_tensors(scheme: str, weight: torch.Tensor) -> dict[str, torch.Tensor]:
    from kairyu_amd.quant import awq, fp8, gptq, int8

    if scheme == "fp8":
        q, s = fp8.quantize_fp8(weight, per_channel=True)
        return {"weight": q, "weight_scale": s}
    if scheme == "int8":
        q, s = int8.quantize_int8_weight(weight)
        return {"weight": q, "weight_scale": s}
    if scheme == "awq":
        q, z, s = awq.quantize_awq(weight, group_size=16)
        return {"qweight": q, "qzeros": z, "scales": s}
    q, z, s, g = gptq.quantize_gptq(weight, group_size=16)
    return {"qweight": q, "qzeros": z, "scales": s, "g_idx": g}


def _quantized_model(scheme: str, device: str, gpu: bool):
    from kairyu_amd.quant.linear import LinearRole, linear_factory, make_linear
    from kairyu_amd.quant.quant_config import detect_quantization

    torch.manual_seed(41)
    model = transformers.LlamaForCausalLM(transformers.LlamaConfig(**TINY)).to(torch.float32).eval()
    quant = detect_quantization({"quantization_config": QUANT_CONFIGS[scheme]})
    factory = linear_factory(quant, device=torch.device(device),
                             dtype=torch.bfloat16 if gpu else torch.float32)
    for index, layer in enumerate(model.model.layers):
        for owner_name, owner in (("self_attn", layer.self_attn), ("mlp", layer.mlp)):
            for name, role in _ROLES.items():
                dense = getattr(owner, name, None)
                if dense is None:
                    continue
                module = make_linear(factory, dense.in_features, dense.out_features, False,
                                     qualified_name=f"model.layers.{index}.{owner_name}.{name}",
                                     role=getattr(LinearRole, role), layer_index=index,
                                     shard_dim=1 if name in ("o_proj", "down_proj") else 0)
                with torch.no_grad():
                    for key, value in _quantized_tensors(scheme, dense.weight.detach()).items():
                        getattr(module, key).copy_(value)
                setattr(owner, name, _Bf16Projection(module) if gpu else module)
    return model.to(device)


def _greedy(model, device: str, prompt, max_new: int = 8) -> list[int]:
    ids = torch.tensor([list(prompt)], device=device)
    out = []
    with torch.no_grad():
        for _ in range(max_new):
            token = int(model(ids).logits[0, -1].argmax())
            out.append(token)
            ids = torch.cat([ids, torch.tensor([[token]], device=device)], dim=1)
    return out


@pytest.mark.parametrize("scheme", ["fp8", "int8", "awq", "gptq"])
def test_quantized_model_generates_on_gpu(cuda, scheme):
    from kairyu_amd.kernels import quant_gemm_hip as hip

    prompt = tuple(range(10))
    cpu_tokens = _greedy(_quantized_model(scheme, "cpu", gpu=False), "cpu", prompt)
    model = _quantized_model(scheme, cuda, gpu=True)
    # the projections run the bound HIP forwards, not a fallback
    first = model.model.layers[0].self_attn.q_proj.inner
    assert first._fused_forward in (hip.fp8_linear_forward, hip.int8_linear_forward,
                                    hip.awq_linear_forward, hip.gptq_linear_forward)
    gpu_tokens = _greedy(model, cuda, prompt)
    print(f"[full model] {scheme} cpu {cpu_tokens} gpu {gpu_tokens}", flush=True)
    assert len(gpu_tokens) == len(cpu_tokens) == 8
    agreement = sum(a == b for a, b in zip(gpu_tokens, cpu_tokens, strict=True)) / len(cpu_tokens)
    assert agreement >= 0.5, f"{scheme}: CPU/GPU greedy agreement {agreement}"
    assert len(set(gpu_tokens)) > 1, f"{scheme}: degenerate output {gpu_tokens}"
