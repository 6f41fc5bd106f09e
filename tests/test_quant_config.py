"""Checkpoint quantization detection and intake (host logic, CPU).

Known answers transcribed from the reference's own tests
(tests/unit/test_quant_config.py:13-246, tests/unit/test_config_and_fp8_load.py:61-151)
against this package's ``detect_quantization`` / ``load_checkpoint_quantization``.
Two deliberate differences, both scope decisions of this package:

* block-wise FP8 (``weight_block_size``) is rejected by the reference
  (test_config_and_fp8_load.py:142-151) and accepted here for ``[128, 128]``
  only (the MoE experts' format), still rejected for every other block;
* NVIDIA's NVFP4 (modelopt ``quant_algo: NVFP4``) is rejected loudly here,
  where the reference detects it; the external-metadata cases therefore use
  ``quant_algo: FP8``.
"""

from __future__ import annotations

import json

import pytest
import torch

from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear
from kairyu_amd.quant.loading import normalize_quantized_state, quantized_buffer_dtypes
from kairyu_amd.quant.quant_config import (
    QuantConfig,
    QuantMethod,
    detect_quantization,
    load_checkpoint_quantization,
)


def test_no_quantization_config_means_none():
    assert detect_quantization({"model_type": "llama"}) == QuantConfig(method=QuantMethod.NONE)


def test_fp8_via_compressed_tensors_is_static_unless_marked_dynamic():
    group = {"weights": {"num_bits": 8, "type": "float"},
             "input_activations": {"num_bits": 8, "type": "float"}}
    config = detect_quantization({"quantization_config": {
        "quant_method": "compressed-tensors", "config_groups": {"group_0": group}}})
    assert config.method is QuantMethod.FP8
    assert (config.weight_bits, config.activation_bits, config.activation_dynamic) == (8, 8, False)
    group["input_activations"]["dynamic"] = True
    config = detect_quantization({"quantization_config": {
        "quant_method": "compressed-tensors", "config_groups": {"group_0": group}}})
    assert config.activation_dynamic is True


def test_int8_via_compressed_tensors():
    config = detect_quantization({"quantization_config": {
        "quant_method": "compressed-tensors",
        "config_groups": {"g": {"weights": {"num_bits": 8, "type": "int"},
                                "input_activations": {"num_bits": 8, "type": "int"}}}}})
    assert config.method is QuantMethod.INT8 and config.weight_bits == 8


def test_compressed_tensors_fp4_is_rejected():
    with pytest.raises(ValueError, match="FP4"):
        detect_quantization({"quantization_config": {
            "quant_method": "compressed-tensors",
            "config_groups": {"g": {"weights": {"num_bits": 4, "type": "float"}}}}})


def test_fp8_direct_method_defaults_to_dynamic():
    config = detect_quantization({"quantization_config": {"quant_method": "fp8"}})
    assert config.method is QuantMethod.FP8 and config.activation_dynamic is True


def test_fp8_static_activation_scheme_is_preserved():
    config = detect_quantization(
        {"quantization_config": {"quant_method": "fp8", "activation_scheme": "static"}})
    assert config.activation_dynamic is False


def test_fp8_unknown_activation_scheme_fails_loudly():
    with pytest.raises(ValueError, match="activation_scheme"):
        detect_quantization(
            {"quantization_config": {"quant_method": "fp8", "activation_scheme": "block"}})


def test_modelopt_fp8_unknown_activation_scheme_fails_loudly():
    with pytest.raises(ValueError, match="modelopt FP8 activation_scheme"):
        detect_quantization({"quantization_config": {
            "quant_method": "modelopt", "quant_algo": "FP8", "activation_scheme": "block"}})


@pytest.mark.parametrize("group_size", [16, 8, 32, "16", True])
def test_modelopt_nvfp4_is_rejected(group_size):
    with pytest.raises(ValueError, match="NVFP4"):
        detect_quantization({"quantization_config": {
            "quant_method": "modelopt", "quant_algo": "NVFP4", "group_size": group_size}})


def test_awq_with_group_size():
    config = detect_quantization(
        {"quantization_config": {"quant_method": "awq", "bits": 4, "group_size": 128}})
    assert (config.method, config.weight_bits, config.group_size) == (QuantMethod.AWQ, 4, 128)


def test_awq_other_than_gemm_layout_is_rejected():
    with pytest.raises(ValueError, match="gemm"):
        detect_quantization({"quantization_config": {"quant_method": "awq", "bits": 4,
                                                     "version": "gemv"}})


def test_gptq():
    config = detect_quantization(
        {"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 128}})
    assert (config.method, config.weight_bits, config.group_size) == (QuantMethod.GPTQ, 4, 128)


@pytest.mark.parametrize("quant,message", [
    ({"bits": 8}, "only 4-bit"),
    ({"bits": 4, "checkpoint_format": "gptq_v2"}, "gptq_v2"),
])
def test_gptq_rejections(quant, message):
    with pytest.raises(ValueError, match=message):
        detect_quantization({"quantization_config": {"quant_method": "gptq", **quant}})


def test_checkpoint_ignore_metadata_is_preserved():
    config = detect_quantization({"quantization_config": {
        "quant_method": "fp8", "ignore": ["lm_head", r"re:model\.layers\.0\..*"]}})
    assert config.ignored_layers == ("lm_head", r"re:model\.layers\.0\..*")


@pytest.mark.parametrize("ignore", ["lm_head", [""]])
def test_malformed_checkpoint_ignore_metadata_fails(ignore):
    with pytest.raises(ValueError, match="ignore"):
        detect_quantization({"quantization_config": {"quant_method": "fp8", "ignore": ignore}})


def test_unsupported_method_raises_with_supported_list():
    with pytest.raises(ValueError, match="awq"):
        detect_quantization({"quantization_config": {"quant_method": "bitsandbytes"}})


# ------------------------------------------------------------ block FP8
def test_block_fp8_128x128_is_accepted():
    config = detect_quantization({"quantization_config": {
        "quant_method": "fp8", "weight_block_size": [128, 128], "activation_scheme": "dynamic"}})
    assert config.method is QuantMethod.FP8_BLOCK
    assert config.weight_block_size == (128, 128) and config.activation_dynamic is True


@pytest.mark.parametrize("block", [[64, 64], [128, 64], [128], "128x128", [128.0, 128.0], [True, 128]])
def test_other_block_sizes_are_rejected_loudly(block):
    with pytest.raises(ValueError, match="block-wise FP8"):
        detect_quantization({"quantization_config": {"quant_method": "fp8",
                                                     "weight_block_size": block}})


def test_block_fp8_requires_dynamic_activations():
    with pytest.raises(ValueError, match="dynamic"):
        detect_quantization({"quantization_config": {
            "quant_method": "fp8", "weight_block_size": [128, 128], "activation_scheme": "static"}})


# ------------------------------------------------- external modelopt metadata
def _write_external_modelopt(path, **quantization):
    (path / "hf_quant_config.json").write_text(json.dumps({
        "producer": {"name": "modelopt", "version": "0.33.0"},
        "quantization": {"quant_algo": "FP8", "exclude_modules": ["model.layers.0.mlp.gate", "lm_head"],
                         **quantization},
    }))


def test_external_modelopt_metadata_is_not_mistaken_for_dense(tmp_path):
    _write_external_modelopt(tmp_path, kv_cache_quant_algo="FP8")
    resolved = load_checkpoint_quantization(tmp_path, {"model_type": "qwen3_moe"})
    assert resolved.weights == QuantConfig(
        method=QuantMethod.FP8, weight_bits=8, activation_bits=8, activation_dynamic=True,
        ignored_layers=("model.layers.0.mlp.gate", "lm_head"))
    assert resolved.source == "hf_quant_config.json"
    assert resolved.kv_cache_quant_algo == "FP8"
    assert (resolved.producer_name, resolved.producer_version) == ("modelopt", "0.33.0")


def test_embedded_metadata_alone_resolves_from_config(tmp_path):
    resolved = load_checkpoint_quantization(
        tmp_path, {"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 128}})
    assert resolved.source == "config.json" and resolved.weights.method is QuantMethod.GPTQ


def test_external_nvfp4_metadata_is_rejected(tmp_path):
    _write_external_modelopt(tmp_path, quant_algo="NVFP4", group_size=16)
    with pytest.raises(ValueError, match="NVFP4"):
        load_checkpoint_quantization(tmp_path, {})


@pytest.mark.parametrize("contents", [
    '{"producer":{"name":"modelopt","name":"other","version":"0.33.0"},"quantization":{}}',
    '{"producer":{"name":"modelopt","version":"0.33.0"},'
    '"quantization":{"quant_algo":"FP8","quant_algo":"FP8"}}',
])
def test_external_modelopt_metadata_rejects_duplicate_json_keys(tmp_path, contents):
    (tmp_path / "hf_quant_config.json").write_text(contents)
    with pytest.raises(ValueError, match="invalid external quantization metadata"):
        load_checkpoint_quantization(tmp_path, {})


@pytest.mark.parametrize("producer", [
    {"name": " ", "version": "0.33.0"},
    {"name": "modelopt", "version": " \t"},
    {"name": "modelopt", "version": " 0.33.0"},
    {"name": "modelopt", "version": "0.33.0 "},
])
def test_external_modelopt_metadata_rejects_whitespace_producer_fields(tmp_path, producer):
    _write_external_modelopt(tmp_path)
    payload = json.loads((tmp_path / "hf_quant_config.json").read_text())
    payload["producer"] = producer
    (tmp_path / "hf_quant_config.json").write_text(json.dumps(payload))
    with pytest.raises(ValueError, match="producer"):
        load_checkpoint_quantization(tmp_path, {})


def test_external_and_embedded_quantization_must_agree(tmp_path):
    _write_external_modelopt(tmp_path)
    embedded = {"quantization_config": {"quant_method": "fp8", "activation_scheme": "static"}}
    with pytest.raises(ValueError, match="disagree"):
        load_checkpoint_quantization(tmp_path, embedded)


@pytest.mark.parametrize(("mutation", "message"), [
    ({"producer": {"name": "other", "version": "1"}}, "producer"),
    ({"quantization": {"quant_algo": "FP8", "exclude_modules": "lm_head"}}, "exclude"),
    ({"quantization": {"quant_algo": "FP8", "exclude_modules": [], "kv_cache_quant_algo": "INT8"}},
     "kv_cache_quant_algo"),
])
def test_external_modelopt_metadata_fails_closed(tmp_path, mutation, message):
    _write_external_modelopt(tmp_path)
    payload = json.loads((tmp_path / "hf_quant_config.json").read_text())
    payload.update(mutation)
    (tmp_path / "hf_quant_config.json").write_text(json.dumps(payload))
    with pytest.raises(ValueError, match=message):
        load_checkpoint_quantization(tmp_path, {})


# ----------------------------------------------------- module intake rules
def test_fp8_linear_loads_per_tensor_scale():
    layer = Fp8Linear(in_features=8, out_features=4, bias=False)
    state = {"weight": torch.zeros(4, 8, dtype=torch.float8_e4m3fn), "weight_scale": torch.tensor([0.5])}
    _, unexpected = layer.load_state_dict(state, strict=False, assign=True)
    assert not unexpected
    assert layer.weight_scale.shape == (1,)
    assert layer.dequantize().shape == (4, 8)


def test_fp8_linear_still_loads_per_channel_scale():
    layer = Fp8Linear(in_features=8, out_features=4, bias=False)
    state = {"weight": torch.zeros(4, 8, dtype=torch.float8_e4m3fn), "weight_scale": torch.ones(4, 1)}
    layer.load_state_dict(state, strict=False, assign=True)
    assert layer.weight_scale.shape == (4, 1)


def test_static_fp8_linear_requires_and_uses_input_scale():
    layer = Fp8Linear(in_features=8, out_features=4, bias=False, activation_dynamic=False)
    state = {"weight": torch.zeros(4, 8, dtype=torch.float8_e4m3fn),
             "weight_scale": torch.tensor([0.5]), "input_scale": torch.tensor(0.25)}
    missing, unexpected = layer.load_state_dict(state, strict=True, assign=True)
    assert not missing and not unexpected
    assert layer.input_scale.item() == 0.25


def test_group_size_minus_one_is_a_single_group():
    awq = AwqLinear(in_features=32, out_features=16, bias=False, group_size=-1)
    assert awq.group_size == 32 and awq.dequantize().shape == (16, 32)
    gptq = GptqLinear(in_features=32, out_features=16, bias=False, group_size=-1)
    assert gptq.group_size == 32 and gptq.dequantize().shape == (16, 32)


def test_invalid_packed_linear_dimensions_fail_at_construction():
    with pytest.raises(ValueError, match="AWQ out_features"):
        AwqLinear(64, 31, bias=False, group_size=16)
    with pytest.raises(ValueError, match="group_size"):
        AwqLinear(72, 32, bias=False, group_size=16)
    with pytest.raises(ValueError, match="GPTQ"):
        GptqLinear(63, 32, bias=False, group_size=16)


def test_quantized_scales_normalize_to_the_kernel_dtype_at_bf16_compute_dtype():
    """A checkpoint may store FP8 per-channel scales in bf16 and W4A16 scales
    in fp32; the quantized buffers keep their registered (kernel ABI) dtype,
    while ordinary fp32 parameters follow the compute dtype (the reference's
    loader rule, kairyu/models/loader.py:219-247)."""
    model = torch.nn.Module()
    model.proj = Fp8Linear(8, 4, bias=True)
    model.awq = AwqLinear(32, 16, bias=False, group_size=16)
    model.norm = torch.nn.LayerNorm(8)
    dtypes = quantized_buffer_dtypes(model)
    assert dtypes["proj.weight_scale"] is torch.float32 and dtypes["awq.scales"] is torch.float16
    assert "proj.bias" not in dtypes   # a parameter, not a packed buffer
    state = {name: t.clone() for name, t in model.state_dict().items()}
    state["proj.weight_scale"] = torch.full((4, 1), 0.5, dtype=torch.bfloat16)
    state["awq.scales"] = torch.full((2, 16), 0.25, dtype=torch.float32)
    out = normalize_quantized_state(model, state, torch.bfloat16)
    assert out["proj.weight_scale"].dtype is torch.float32
    assert torch.equal(out["proj.weight_scale"], torch.full((4, 1), 0.5))
    assert out["awq.scales"].dtype is torch.float16
    assert out["proj.weight"].dtype is torch.float8_e4m3fn
    assert out["proj.bias"].dtype is torch.bfloat16 and out["norm.weight"].dtype is torch.bfloat16
    model.load_state_dict(out, strict=True, assign=True)
    assert model.proj.weight_scale.dtype is torch.float32


def test_validate_model_quantization_rejects_quantized_mla():
    """kairyu/engine/core/quant_config.py:308-321: a quantized checkpoint is
    refused for an MLA architecture before the model is built; dense MLA and
    quantized non-MLA models pass."""
    from kairyu_amd.quant.quant_config import QuantConfig, QuantMethod, validate_model_quantization

    fp8 = detect_quantization({"quantization_config": {"quant_method": "fp8"}})
    with pytest.raises(ValueError, match="DeepseekV3ForCausalLM MLA does not support fp8 checkpoints: "
                                         "its absorbed KV projection requires an unquantized kv_b_proj weight"):
        validate_model_quantization(fp8, is_mla=True, architecture="DeepseekV3ForCausalLM")
    validate_model_quantization(fp8, is_mla=False, architecture="LlamaForCausalLM")
    validate_model_quantization(QuantConfig(method=QuantMethod.NONE), is_mla=True,
                                architecture="DeepseekV3ForCausalLM")
