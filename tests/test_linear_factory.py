"""Construction-time contracts of the contextual linear factory (host logic, CPU).

Transcribed from the reference's tests/unit/test_linear_factory_context.py
(:225-275 selection and kernel binding, :322-410 error text, exclusions and
dense-by-role, :466 the legacy three-argument factory) onto this package's
``linear_factory`` / ``make_linear``, with the gfx950 HIP kernel families in
place of the reference's CUDA ones.  The model-zoo constructions of the
reference's tests (``DenseDecoder``, draft heads, loaders) are out of this
package's scope, so projections are built with ``make_linear`` directly under
the same names, roles and placements.
"""

from __future__ import annotations

import pytest
import torch

from kairyu_amd.kernels import quant_gemm_hip as hip
from kairyu_amd.quant.linear import (
    AwqLinear,
    BlockFp8Linear,
    ExpertScope,
    Fp8Linear,
    GptqLinear,
    Int8Linear,
    LinearKernel,
    LinearKernelCapabilities,
    LinearRole,
    LinearSelection,
    TensorParallelMode,
    linear_factory,
    make_linear,
)
from kairyu_amd.quant.quant_config import QuantConfig, QuantMethod, detect_quantization

_HIP_ALL = LinearKernelCapabilities(
    frozenset({LinearKernel.TORCH_DENSE, LinearKernel.HIP_FP8_W8A8, LinearKernel.HIP_INT8_W8A8,
               LinearKernel.HIP_W4A16, LinearKernel.HIP_FP8_BLOCK}),
    "test-gfx950",
)


def _q_proj(factory, **kw):
    return make_linear(factory, 32, 16, False, qualified_name=kw.pop("name", "model.layers.4.self_attn.q_proj"),
                       role=kw.pop("role", LinearRole.ATTENTION_QUERY), layer_index=4, shard_dim=0, **kw)


def test_specialized_policy_selects_format_by_context():
    def policy(_checkpoint_quant, context):
        if context.role is LinearRole.ATTENTION_QUERY:
            quant = QuantConfig(QuantMethod.FP8, weight_bits=8)
        elif context.role is LinearRole.MLP_UP:
            quant = QuantConfig(QuantMethod.INT8, weight_bits=8)
        else:
            quant = QuantConfig(QuantMethod.NONE)
        return LinearSelection(quant, None, f"role:{context.role.value}")

    factory = linear_factory(QuantConfig(QuantMethod.NONE), selection_policy=policy)
    q = make_linear(factory, 32, 32, False, qualified_name="model.layers.0.self_attn.q_proj",
                    role=LinearRole.ATTENTION_QUERY, layer_index=0, shard_dim=0)
    up = make_linear(factory, 32, 64, False, qualified_name="model.layers.0.mlp.up_proj",
                     role=LinearRole.MLP_UP, layer_index=0, shard_dim=0)
    k = make_linear(factory, 32, 16, False, qualified_name="model.layers.0.self_attn.k_proj",
                    role=LinearRole.ATTENTION_KEY, layer_index=0, shard_dim=0)
    assert isinstance(q, Fp8Linear) and isinstance(up, Int8Linear)
    assert type(k) is torch.nn.Linear
    assert up.linear_selection.reason == "role:mlp_up"
    assert up.linear_selection.kernel is LinearKernel.CPU_REFERENCE
    assert not hasattr(up, "_fused_forward")          # host kernels bind nothing


@pytest.mark.parametrize("quant,cls,forward", [
    (QuantConfig(QuantMethod.FP8), Fp8Linear, "fp8_linear_forward"),
    (QuantConfig(QuantMethod.INT8), Int8Linear, "int8_linear_forward"),
    (QuantConfig(QuantMethod.AWQ, weight_bits=4, group_size=16), AwqLinear, "awq_linear_forward"),
    (QuantConfig(QuantMethod.GPTQ, weight_bits=4, group_size=16), GptqLinear, "gptq_linear_forward"),
    (QuantConfig(QuantMethod.FP8_BLOCK, weight_block_size=(128, 128)), BlockFp8Linear,
     "block_fp8_linear_forward"),
])
def test_device_kernel_is_bound_from_the_selected_kernel_family(quant, cls, forward):
    module = _q_proj(linear_factory(quant, device="cuda:3", dtype=torch.bfloat16, capabilities=_HIP_ALL))
    assert isinstance(module, cls)
    assert module.linear_selection.kernel is _HIP_ALL.preferred_kernel(quant.method)
    assert module._fused_forward is getattr(hip, forward)
    assert module._fused_forward.__name__ == forward


def test_unsupported_context_error_is_deterministic_and_actionable():
    capabilities = LinearKernelCapabilities(frozenset({LinearKernel.TORCH_DENSE}), "test-gfx942-no-lib")
    factory = linear_factory(QuantConfig(QuantMethod.FP8), device="cuda:3", dtype=torch.bfloat16,
                             tensor_parallel_size=4, tensor_parallel_rank=2, capabilities=capabilities)
    messages = []
    for _ in range(2):
        with pytest.raises(RuntimeError) as caught:
            make_linear(factory, 32, 16, False, qualified_name="model.layers.9.self_attn.q_proj",
                        role=LinearRole.ATTENTION_QUERY, layer_index=9, shard_dim=0)
        messages.append(str(caught.value))
    assert messages[0] == messages[1]
    message = messages[0]
    for part in ("no production kernel for fp8", "name='model.layers.9.self_attn.q_proj'",
                 "role=attention_query", "device=cuda:3", "dtype=torch.bfloat16",
                 "tp=column:2/4:dim=0", "local=32x16, global=32x64",
                 "capabilities=test-gfx942-no-lib"):
        assert part in message, part


def test_host_kernel_on_a_device_target_and_float32_device_compute_are_rejected():
    cpu_only = LinearKernelCapabilities(
        frozenset({LinearKernel.TORCH_DENSE, LinearKernel.CPU_REFERENCE}), "test-host")
    with pytest.raises(RuntimeError, match="incompatible with target cuda"):
        _q_proj(linear_factory(QuantConfig(QuantMethod.FP8), device="cuda:0", dtype=torch.bfloat16,
                               capabilities=cpu_only))
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        _q_proj(linear_factory(QuantConfig(QuantMethod.FP8), device="cuda:0", dtype=torch.float32,
                               capabilities=_HIP_ALL))


def test_architectural_exclusion_cannot_be_overridden():
    default = make_linear(linear_factory(QuantConfig(QuantMethod.FP8)), 32, 16, False,
                          qualified_name="model.layers.0.self_attn.kv_b_proj",
                          role=LinearRole.MLA_KV_B, allow_quantization=False)
    assert type(default) is torch.nn.Linear
    assert default.linear_selection.reason == "architectural-exclusion"

    def invalid_policy(_checkpoint_quant, _context):
        return LinearSelection(QuantConfig(QuantMethod.FP8), LinearKernel.CPU_REFERENCE, "invalid-override")

    with pytest.raises(ValueError, match="excludes quantization"):
        make_linear(linear_factory(QuantConfig(QuantMethod.NONE), selection_policy=invalid_policy),
                    32, 16, False, qualified_name="model.layers.0.self_attn.kv_b_proj",
                    role=LinearRole.MLA_KV_B, allow_quantization=False)


@pytest.mark.parametrize("role", [LinearRole.MOE_ROUTER, LinearRole.OUTPUT_HEAD, LinearRole.DRAFT_FUSION])
def test_accuracy_sensitive_roles_default_to_dense(role):
    module = make_linear(linear_factory(QuantConfig(QuantMethod.FP8)), 32, 16, False,
                         qualified_name=f"test.{role.value}", role=role)
    assert type(module) is torch.nn.Linear
    assert module.linear_selection.reason == f"default-dense-role:{role.value}"


def test_checkpoint_exclusions_are_dense():
    quant = detect_quantization({"quantization_config": {
        "quant_method": "compressed-tensors",
        "config_groups": {"group_0": {"weights": {"type": "float", "num_bits": 8},
                                      "input_activations": {"type": "float", "num_bits": 8,
                                                            "dynamic": True}}},
        "ignore": ["model.layers.0.self_attn.q_proj", r"re:model\.layers\.0\.mlp\.(gate|up)_proj"],
    }})
    factory = linear_factory(quant)

    def build(name, role):
        return make_linear(factory, 32, 32, False, qualified_name=name, role=role, layer_index=0)

    q = build("model.layers.0.self_attn.q_proj", LinearRole.ATTENTION_QUERY)
    gate = build("model.layers.0.mlp.gate_proj", LinearRole.MLP_GATE)
    up = build("model.layers.0.mlp.up_proj", LinearRole.MLP_UP)
    k = build("model.layers.0.self_attn.k_proj", LinearRole.ATTENTION_KEY)
    down = build("model.layers.0.mlp.down_proj", LinearRole.MLP_DOWN)
    assert all(type(m) is torch.nn.Linear for m in (q, gate, up))
    assert isinstance(k, Fp8Linear) and isinstance(down, Fp8Linear)
    assert q.linear_selection.reason == "checkpoint-ignore:model.layers.0.self_attn.q_proj"
    assert k.activation_dynamic is True


def test_placement_and_expert_identity_are_recorded():
    factory = linear_factory(QuantConfig(QuantMethod.FP8_BLOCK), device="cuda:1", dtype=torch.bfloat16,
                             tensor_parallel_size=2, tensor_parallel_rank=1, capabilities=_HIP_ALL)
    up = make_linear(factory, 2048, 384, False, qualified_name="model.layers.3.mlp.experts.5.up_proj",
                     role=LinearRole.MLP_UP, layer_index=3, expert_index=5,
                     expert_scope=ExpertScope.ROUTED, shard_dim=0)
    down = make_linear(factory, 384, 2048, False, qualified_name="model.layers.3.mlp.experts.5.down_proj",
                       role=LinearRole.MLP_DOWN, layer_index=3, expert_index=5,
                       expert_scope=ExpertScope.ROUTED, shard_dim=1)
    ctx = up.linear_context
    assert (ctx.expert_index, ctx.expert_scope, ctx.layer_index) == (5, ExpertScope.ROUTED, 3)
    assert ctx.tensor_parallel.mode is TensorParallelMode.COLUMN
    assert (ctx.tensor_parallel.local_out_features, ctx.tensor_parallel.global_out_features) == (384, 768)
    assert down.linear_context.tensor_parallel.mode is TensorParallelMode.ROW
    assert down.linear_context.tensor_parallel.global_in_features == 768
    with pytest.raises(ValueError, match="expert_index"):
        make_linear(factory, 32, 32, False, qualified_name="x", role=LinearRole.MLP_UP,
                    expert_scope=ExpertScope.ROUTED)


def test_legacy_three_argument_factory_remains_compatible():
    calls = []

    def legacy(in_features, out_features, bias):
        calls.append((in_features, out_features, bias))
        return torch.nn.Linear(in_features, out_features, bias=bias)

    built = make_linear(legacy, 32, 16, True, qualified_name="model.layers.0.self_attn.q_proj",
                        role=LinearRole.ATTENTION_QUERY)
    assert calls == [(32, 16, True)] and type(built) is torch.nn.Linear
    direct = linear_factory(QuantConfig(QuantMethod.FP8))(32, 16, False)
    assert isinstance(direct, Fp8Linear)
    assert not hasattr(direct, "linear_context")


def test_capabilities_for_the_host_and_other_device_types():
    cpu = LinearKernelCapabilities.for_device("cpu")
    assert cpu.available_kernels == frozenset({LinearKernel.TORCH_DENSE, LinearKernel.CPU_REFERENCE})
    assert cpu.preferred_kernel(QuantMethod.GPTQ) is LinearKernel.CPU_REFERENCE
    assert cpu.preferred_kernel(QuantMethod.NONE) is LinearKernel.TORCH_DENSE
    meta = LinearKernelCapabilities.for_device("meta")
    assert meta.supported_quant_methods == frozenset({QuantMethod.NONE})
    assert _HIP_ALL.preferred_kernel(QuantMethod.AWQ) is LinearKernel.HIP_W4A16
    with pytest.raises(ValueError, match="torch_dense"):
        LinearKernelCapabilities(frozenset({LinearKernel.HIP_W4A16}), "x")


def test_legacy_per_format_modules_forward_to_the_fused_kernels(monkeypatch):
    from kairyu_amd.kernels import awq_gemm_hip, fp8_gemm_hip, gptq_gemm_hip, int8_gemm_hip

    seen = []
    for name, module in (("awq", awq_gemm_hip), ("gptq", gptq_gemm_hip), ("fp8", fp8_gemm_hip),
                         ("int8", int8_gemm_hip)):
        assert module._forward is getattr(hip, f"{name}_linear_forward")
        monkeypatch.setattr(module, "_forward", lambda x, m, _n=name: seen.append((_n, x, m)) or _n)
        assert module.linear_forward("x", "module") == name
    assert seen == [(n, "x", "module") for n in ("awq", "gptq", "fp8", "int8")]


def test_checkpoint_member_layout_binding():
    """``bind_checkpoint_member_layout`` (kairyu/quant/linear.py:101-119),
    as the reference's MoE router binds its ``e_score_correction_bias``
    (kairyu/models/moe.py:372-376): a direct member gets one layout; dotted
    names, unregistered members and a second binding are rejected."""

    from kairyu_amd.quant.linear import CheckpointMemberLayout, bind_checkpoint_member_layout

    gate = torch.nn.Linear(16, 8, bias=False)
    gate.register_buffer("e_score_correction_bias", torch.zeros(8))
    layout = CheckpointMemberLayout(column_dim=0, row_dim=None)
    bind_checkpoint_member_layout(gate, "e_score_correction_bias", layout)
    assert gate._kairyu_checkpoint_member_layouts == {"e_score_correction_bias": layout}
    assert layout.shard_dim(TensorParallelMode.COLUMN) == 0
    assert layout.shard_dim(TensorParallelMode.ROW) is None
    with pytest.raises(ValueError, match="already has a layout"):
        bind_checkpoint_member_layout(gate, "e_score_correction_bias", layout)
    with pytest.raises(ValueError, match="direct member name"):
        bind_checkpoint_member_layout(gate, "inner.bias", layout)
    with pytest.raises(ValueError, match="not registered directly"):
        bind_checkpoint_member_layout(gate, "missing", layout)
    with pytest.raises(ValueError, match="shard dim"):
        CheckpointMemberLayout(column_dim=2, row_dim=None)
