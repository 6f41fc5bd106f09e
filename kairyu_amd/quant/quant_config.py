"""HF ``quantization_config`` -> :class:`QuantConfig` detection.

Interface of kairyu/engine/core/quant_config.py:27-295 (``QuantMethod``,
``QuantConfig``, ``CheckpointQuantization``, ``detect_quantization``,
``load_checkpoint_quantization``), limited to the formats this
package executes on gfx950: FP8 (per-tensor / per-channel), INT8 W8A8, AWQ and
GPTQ W4A16, plus 128x128 block-scaled FP8 (``weight_block_size``), which the
reference rejects (quant_config.py:156-163) and this package adds as its own
method for block-scaled MoE experts.  NVFP4 / ModelOpt FP4 checkpoints are
rejected loudly: that NVIDIA FP4 ABI is not part of this package.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from enum import Enum
from pathlib import Path


class QuantMethod(Enum):
    NONE = "none"
    FP8 = "fp8"
    INT8 = "int8"
    AWQ = "awq"
    GPTQ = "gptq"
    FP8_BLOCK = "fp8_block"


_SUPPORTED = (
    QuantMethod.FP8,
    QuantMethod.INT8,
    QuantMethod.AWQ,
    QuantMethod.GPTQ,
    QuantMethod.FP8_BLOCK,
)

SUPPORTED_WEIGHT_BLOCK = (128, 128)


@dataclass(frozen=True)
class QuantConfig:
    method: QuantMethod
    weight_bits: int | None = None
    activation_bits: int | None = None
    group_size: int | None = None
    activation_dynamic: bool | None = None
    ignored_layers: tuple[str, ...] = ()
    weight_block_size: tuple[int, int] | None = None


@dataclass(frozen=True)
class CheckpointQuantization:
    """Resolved weight metadata for one local HF checkpoint."""

    weights: QuantConfig
    source: str
    kv_cache_quant_algo: str | None = None
    producer_name: str | None = None
    producer_version: str | None = None


def _unique_keys(pairs: list[tuple[str, object]]) -> dict[str, object]:
    result: dict[str, object] = {}
    for key, value in pairs:
        if key in result:
            raise ValueError(f"duplicate JSON key {key!r}")
        result[key] = value
    return result


def _ignored_layers(quant: dict) -> tuple[str, ...]:
    raw = quant.get("ignore", ())
    if raw is None:
        return ()
    if not isinstance(raw, (list, tuple)) or not all(
        isinstance(item, str) and item for item in raw
    ):
        raise ValueError("quantization ignore must contain non-empty strings")
    return tuple(raw)


def _activation_scheme(quant: dict, label: str) -> bool:
    scheme = str(quant.get("activation_scheme", "dynamic")).lower()
    if scheme not in ("dynamic", "static"):
        raise ValueError(
            f"unsupported {label} activation_scheme {scheme!r}: supported: dynamic, static"
        )
    return scheme == "dynamic"


def _compressed_tensors(quant: dict) -> QuantConfig:
    groups = quant.get("config_groups", {}) or {}
    first = next(iter(groups.values()), {}) or {}
    weights = first.get("weights", {}) or {}
    activations = first.get("input_activations", {}) or {}
    kind, bits = weights.get("type"), weights.get("num_bits")
    if kind == "float" and bits == 8:
        return QuantConfig(
            method=QuantMethod.FP8,
            weight_bits=8,
            activation_bits=activations.get("num_bits"),
            activation_dynamic=bool(activations.get("dynamic", False)),
            ignored_layers=_ignored_layers(quant),
        )
    if kind == "int" and bits == 8:
        return QuantConfig(
            method=QuantMethod.INT8,
            weight_bits=8,
            activation_bits=activations.get("num_bits"),
            ignored_layers=_ignored_layers(quant),
        )
    if kind == "float" and bits == 4:
        raise ValueError("compressed-tensors FP4 checkpoints are not supported")
    raise ValueError("unsupported compressed-tensors scheme: FP8/INT8 W8A8 are supported")


def _modelopt(quant: dict) -> QuantConfig:
    algo = str(quant.get("quant_algo", "")).upper()
    if algo == "FP8":
        return QuantConfig(
            method=QuantMethod.FP8,
            weight_bits=8,
            activation_bits=8,
            activation_dynamic=_activation_scheme(quant, "modelopt FP8"),
            ignored_layers=_ignored_layers(quant),
        )
    if algo == "NVFP4":
        raise ValueError(
            "modelopt NVFP4 checkpoints are not supported: NVFP4 is an NVIDIA FP4 ABI with no "
            "gfx950 kernel in this package; supported modelopt quant_algo: FP8"
        )
    raise ValueError(f"unsupported modelopt quant_algo {algo!r}; supported: FP8")


def _block_fp8(quant: dict) -> QuantConfig:
    block = quant.get("weight_block_size")
    if (
        not isinstance(block, (list, tuple))
        or len(block) != 2
        or any(type(value) is not int for value in block)
        or tuple(block) != SUPPORTED_WEIGHT_BLOCK
    ):
        raise ValueError(
            f"unsupported block-wise FP8 weight_block_size {block!r}; supported: [128, 128]"
        )
    if not _activation_scheme(quant, "block FP8"):
        raise ValueError("block-wise FP8 requires dynamic activation quantization")
    return QuantConfig(
        method=QuantMethod.FP8_BLOCK,
        weight_bits=8,
        activation_bits=8,
        activation_dynamic=True,
        ignored_layers=_ignored_layers(quant),
        weight_block_size=SUPPORTED_WEIGHT_BLOCK,
    )


def detect_quantization(hf_config: dict) -> QuantConfig:
    quant = hf_config.get("quantization_config")
    if not quant:
        return QuantConfig(method=QuantMethod.NONE)
    method = str(quant.get("quant_method", "")).lower()
    if method == "compressed-tensors":
        return _compressed_tensors(quant)
    if method == "modelopt":
        return _modelopt(quant)
    if method == "fp8":
        if quant.get("weight_block_size") is not None:
            return _block_fp8(quant)
        return QuantConfig(
            method=QuantMethod.FP8,
            weight_bits=8,
            activation_bits=8,
            activation_dynamic=_activation_scheme(quant, "FP8"),
            ignored_layers=_ignored_layers(quant),
        )
    if method == "awq":
        version = str(quant.get("version", "gemm")).lower()
        if version != "gemm":
            raise ValueError(f"unsupported AWQ version {version!r}: only 'gemm' layout is supported")
        return QuantConfig(
            method=QuantMethod.AWQ,
            weight_bits=quant.get("bits"),
            group_size=quant.get("group_size"),
            ignored_layers=_ignored_layers(quant),
        )
    if method == "gptq":
        if quant.get("bits") != 4:
            raise ValueError(f"unsupported GPTQ bits={quant.get('bits')}: only 4-bit")
        if str(quant.get("checkpoint_format", "gptq")).lower() == "gptq_v2":
            raise ValueError(
                "gptq_v2 checkpoints are not supported (v2 drops the zero-point storage "
                "offset; loading as v1 would shift every zero by 1)"
            )
        return QuantConfig(
            method=QuantMethod.GPTQ,
            weight_bits=quant.get("bits"),
            group_size=quant.get("group_size"),
            ignored_layers=_ignored_layers(quant),
        )
    supported = ", ".join(m.value for m in _SUPPORTED)
    raise ValueError(f"unsupported quant_method {method!r}; supported: {supported}")


def load_checkpoint_quantization(model_dir: str | Path, hf_config: dict) -> CheckpointQuantization:
    """Resolve embedded or ModelOpt-external (``hf_quant_config.json``) metadata.

    Both forms must agree when both are present; a mismatch is an error, never
    a silent preference (quant_config.py:206-295).
    """

    directory = Path(model_dir)
    external_path = directory / "hf_quant_config.json"
    embedded = detect_quantization(hf_config)
    if not external_path.is_file():
        return CheckpointQuantization(weights=embedded, source="config.json")
    try:
        payload = json.loads(external_path.read_text(), object_pairs_hook=_unique_keys)
    except (OSError, json.JSONDecodeError, ValueError) as error:
        raise ValueError(f"invalid external quantization metadata at {external_path}") from error
    if not isinstance(payload, dict):
        raise ValueError("hf_quant_config.json must contain a JSON object")
    producer = payload.get("producer")
    quantization = payload.get("quantization")
    if not isinstance(producer, dict) or not isinstance(quantization, dict):
        raise ValueError("hf_quant_config.json requires object-valued producer and quantization")
    name, version = producer.get("name"), producer.get("version")
    if name != "modelopt" or not isinstance(version, str) or not version or version.strip() != version:
        raise ValueError("hf_quant_config.json requires producer name 'modelopt' and a version")
    excludes = quantization.get("exclude_modules", ())
    if not isinstance(excludes, (list, tuple)) or not all(
        isinstance(item, str) and item for item in excludes
    ):
        raise ValueError("hf_quant_config.json exclude_modules must contain non-empty strings")
    external = detect_quantization(
        {
            "quantization_config": {
                "quant_method": "modelopt",
                "quant_algo": quantization.get("quant_algo"),
                "ignore": list(excludes),
            }
        }
    )
    if embedded.method is not QuantMethod.NONE and embedded != external:
        raise ValueError("config.json and hf_quant_config.json quantization metadata disagree")
    raw_kv = quantization.get("kv_cache_quant_algo")
    kv_algo = None if raw_kv is None else str(raw_kv).upper()
    if kv_algo not in (None, "FP8"):
        raise ValueError(f"unsupported ModelOpt kv_cache_quant_algo {raw_kv!r}; supported metadata: FP8")
    return CheckpointQuantization(
        weights=external,
        source="config.json+hf_quant_config.json"
        if embedded.method is not QuantMethod.NONE
        else "hf_quant_config.json",
        kv_cache_quant_algo=kv_algo,
        producer_name=name,
        producer_version=version,
    )


def validate_model_quantization(quant: QuantConfig, *, is_mla: bool, architecture: str) -> None:
    """Reject quantization combinations before the model is built
    (kairyu/engine/core/quant_config.py:308-321, called by the reference's
    loader at kairyu/models/loader.py:186): an MLA architecture's absorbed KV
    projection needs an unquantized ``kv_b_proj`` weight, so any quantized
    checkpoint is refused for it, with the reference's message."""

    if is_mla and quant.method is not QuantMethod.NONE:
        raise ValueError(
            f"{architecture} MLA does not support {quant.method.value} "
            "checkpoints: its absorbed KV projection requires an unquantized "
            "kv_b_proj weight"
        )
