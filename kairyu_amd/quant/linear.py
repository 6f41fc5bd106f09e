"""Quantized linear modules and the contextual linear factory.

Interface of kairyu/quant/linear.py:27-1197 (module classes, buffer ABI,
``linear_factory`` / ``make_linear`` / selection policy / kernel binding),
re-targeted at gfx950: the CUDA-SM capability floors and Triton/FlashInfer
kernel families become one probe of the device's ``gcnArchName`` plus the
presence of this package's HIP library, and quantized device forwards bind to
:mod:`kairyu_amd.kernels.quant_gemm_hip`.

Packed tensors are persistent buffers under the checkpoint's own names, so a
loader assigns them by name.  On a CPU tensor ``forward`` runs the explicit
dequantize-then-matmul path of the reference's ``CPU_REFERENCE`` kernel family;
on a device tensor it runs the bound HIP kernel and never dequantizes the
weight, with no fallback of any kind.
"""

from __future__ import annotations

import inspect
import re
from collections.abc import Callable
from dataclasses import dataclass
from enum import Enum
from typing import Protocol

import torch
from torch import nn

from . import awq, block_fp8, fp8, gptq, int8
from .quant_config import QuantConfig, QuantMethod


class LinearRole(Enum):
    ATTENTION_QUERY = "attention_query"
    ATTENTION_KEY = "attention_key"
    ATTENTION_VALUE = "attention_value"
    ATTENTION_OUTPUT = "attention_output"
    MLA_QUERY_A = "mla_query_a"
    MLA_QUERY_B = "mla_query_b"
    MLA_KV_A = "mla_kv_a"
    MLA_KV_B = "mla_kv_b"
    MLP_GATE = "mlp_gate"
    MLP_UP = "mlp_up"
    MLP_DOWN = "mlp_down"
    MOE_ROUTER = "moe_router"
    DRAFT_FUSION = "draft_fusion"
    OUTPUT_HEAD = "output_head"


class ExpertScope(Enum):
    NONE = "none"
    ROUTED = "routed"
    SHARED = "shared"


class ModelScope(Enum):
    TARGET = "target"
    EAGLE_DRAFT = "eagle_draft"
    MTP_DRAFT = "mtp_draft"


class TensorParallelMode(Enum):
    REPLICATED = "replicated"
    COLUMN = "column"
    ROW = "row"


@dataclass(frozen=True)
class CheckpointMemberLayout:
    """Physical checkpoint axes (column / row TP shard dims) of one member."""

    column_dim: int | None
    row_dim: int | None

    def __post_init__(self) -> None:
        for label, dim in (("column", self.column_dim), ("row", self.row_dim)):
            if dim not in (None, 0, 1):
                raise ValueError(f"{label} checkpoint shard dim must be 0, 1, or None")

    def shard_dim(self, mode: TensorParallelMode) -> int | None:
        if mode is TensorParallelMode.COLUMN:
            return self.column_dim
        if mode is TensorParallelMode.ROW:
            return self.row_dim
        return None


def bind_checkpoint_member_layout(
    module: nn.Module, member: str, layout: CheckpointMemberLayout
) -> None:
    if not member or "." in member:
        raise ValueError("checkpoint member layout requires a direct member name")
    if member not in module._parameters and member not in module._buffers:
        raise ValueError(
            f"checkpoint member {member!r} is not registered directly on {type(module).__name__}"
        )
    layouts = dict(getattr(module, "_kairyu_checkpoint_member_layouts", {}))
    if member in layouts:
        raise ValueError(f"checkpoint member {member!r} already has a layout")
    layouts[member] = layout
    object.__setattr__(module, "_kairyu_checkpoint_member_layouts", layouts)


_EXPECTED_SHARD_DIM = {
    TensorParallelMode.REPLICATED: None,
    TensorParallelMode.COLUMN: 0,
    TensorParallelMode.ROW: 1,
}


@dataclass(frozen=True)
class TensorParallelPlacement:
    mode: TensorParallelMode
    world_size: int
    rank: int
    shard_dim: int | None
    global_in_features: int
    global_out_features: int
    local_in_features: int
    local_out_features: int

    def __post_init__(self) -> None:
        if self.world_size < 1:
            raise ValueError("tensor-parallel world_size must be positive")
        if not 0 <= self.rank < self.world_size:
            raise ValueError(
                f"tensor-parallel rank {self.rank} is outside world_size {self.world_size}"
            )
        if self.shard_dim not in (None, 0, 1):
            raise ValueError("tensor-parallel shard_dim must be 0, 1, or None")
        expected = _EXPECTED_SHARD_DIM[self.mode]
        if self.shard_dim != expected:
            raise ValueError(f"tensor-parallel mode {self.mode.value} requires shard_dim={expected}")
        dims = (
            self.global_in_features,
            self.global_out_features,
            self.local_in_features,
            self.local_out_features,
        )
        if min(dims) < 1:
            raise ValueError("tensor-parallel projection dimensions must be positive")


class LinearKernel(Enum):
    """Kernel family bound to one constructed projection."""

    TORCH_DENSE = "torch_dense"
    CPU_REFERENCE = "cpu_reference"
    HIP_FP8_W8A8 = "hip_fp8_w8a8"
    HIP_INT8_W8A8 = "hip_int8_w8a8"
    HIP_W4A16 = "hip_w4a16"
    HIP_FP8_BLOCK = "hip_fp8_block"


_KERNEL_METHODS: dict[LinearKernel, frozenset[QuantMethod]] = {
    LinearKernel.TORCH_DENSE: frozenset({QuantMethod.NONE}),
    LinearKernel.CPU_REFERENCE: frozenset(
        {
            QuantMethod.FP8,
            QuantMethod.INT8,
            QuantMethod.AWQ,
            QuantMethod.GPTQ,
            QuantMethod.FP8_BLOCK,
        }
    ),
    LinearKernel.HIP_FP8_W8A8: frozenset({QuantMethod.FP8}),
    LinearKernel.HIP_INT8_W8A8: frozenset({QuantMethod.INT8}),
    LinearKernel.HIP_W4A16: frozenset({QuantMethod.AWQ, QuantMethod.GPTQ}),
    LinearKernel.HIP_FP8_BLOCK: frozenset({QuantMethod.FP8_BLOCK}),
}

_PREFERENCE = (
    LinearKernel.TORCH_DENSE,
    LinearKernel.HIP_FP8_W8A8,
    LinearKernel.HIP_INT8_W8A8,
    LinearKernel.HIP_W4A16,
    LinearKernel.HIP_FP8_BLOCK,
    LinearKernel.CPU_REFERENCE,
)

REQUIRED_ARCH = "gfx950"


def _device_arch(device: torch.device) -> str:
    """``gcnArchName`` of a ROCm device (e.g. ``gfx950:sramecc+:xnack-``)."""

    index = device.index if device.index is not None else torch.cuda.current_device()
    return str(torch.cuda.get_device_properties(index).gcnArchName)


def _probe_native_library() -> tuple[bool, str]:
    try:
        from kairyu_amd import _native

        _native.library()
    except RuntimeError as error:
        return False, f"missing:{error}"
    return True, "available"


@dataclass(frozen=True)
class LinearKernelCapabilities:
    """Quantized formats accepted by the target kernel profile.

    Dense construction is always available; quantized formats never fall back
    to dense when a target lacks their kernel.
    """

    available_kernels: frozenset[LinearKernel]
    source: str

    def __post_init__(self) -> None:
        if LinearKernel.TORCH_DENSE not in self.available_kernels:
            raise ValueError("linear capabilities must include torch_dense")
        if not self.source:
            raise ValueError("linear capability source must be non-empty")

    @property
    def supported_quant_methods(self) -> frozenset[QuantMethod]:
        methods: set[QuantMethod] = set()
        for kernel in self.available_kernels:
            methods |= _KERNEL_METHODS[kernel]
        return frozenset(methods)

    def preferred_kernel(self, method: QuantMethod) -> LinearKernel | None:
        for kernel in _PREFERENCE:
            if kernel in self.available_kernels and method in _KERNEL_METHODS[kernel]:
                return kernel
        return None

    @classmethod
    def for_device(cls, device: str | torch.device) -> LinearKernelCapabilities:
        target = torch.device(device)
        if target.type == "cpu":
            return cls(
                frozenset({LinearKernel.TORCH_DENSE, LinearKernel.CPU_REFERENCE}),
                "cpu-reference",
            )
        if target.type != "cuda":
            return cls(frozenset({LinearKernel.TORCH_DENSE}), f"{target.type}-dense-only")
        if not torch.cuda.is_available():
            raise RuntimeError(f"cannot probe linear kernels for {target}: no ROCm device")
        arch = _device_arch(target)
        has_lib, lib_status = _probe_native_library()
        kernels = {LinearKernel.TORCH_DENSE}
        if arch.split(":")[0] == REQUIRED_ARCH and has_lib:
            kernels |= {
                LinearKernel.HIP_FP8_W8A8,
                LinearKernel.HIP_INT8_W8A8,
                LinearKernel.HIP_W4A16,
                LinearKernel.HIP_FP8_BLOCK,
            }
        return cls(frozenset(kernels), f"rocm-{arch.split(':')[0]};hip_lib={lib_status}")


@dataclass(frozen=True)
class LinearBuildContext:
    qualified_name: str
    model_scope: ModelScope
    role: LinearRole
    device: torch.device
    dtype: torch.dtype
    tensor_parallel: TensorParallelPlacement
    capabilities: LinearKernelCapabilities
    layer_index: int | None = None
    expert_index: int | None = None
    expert_scope: ExpertScope = ExpertScope.NONE
    allow_quantization: bool = True

    def __post_init__(self) -> None:
        if not self.qualified_name:
            raise ValueError("linear qualified_name must be non-empty")
        if self.layer_index is not None and self.layer_index < 0:
            raise ValueError("linear layer_index must be non-negative")
        if self.expert_index is not None and self.expert_index < 0:
            raise ValueError("linear expert_index must be non-negative")
        routed = self.expert_scope is ExpertScope.ROUTED
        if routed and self.expert_index is None:
            raise ValueError("routed expert context requires a global expert_index")
        if not routed and self.expert_index is not None:
            raise ValueError(f"{self.expert_scope.value} expert context cannot carry expert_index")


@dataclass(frozen=True)
class LinearSelection:
    quantization: QuantConfig
    kernel: LinearKernel | None
    reason: str
    observe_activation_saturation: bool = False

    def __post_init__(self) -> None:
        if not self.reason:
            raise ValueError("linear selection reason must be non-empty")
        if type(self.observe_activation_saturation) is not bool:
            raise TypeError("activation saturation observation must be a boolean")


LinearSelectionPolicy = Callable[[QuantConfig, LinearBuildContext], LinearSelection]


class LinearFactory(Protocol):
    def __call__(
        self,
        in_features: int,
        out_features: int,
        bias: bool,
        *,
        qualified_name: str,
        model_scope: ModelScope = ModelScope.TARGET,
        role: LinearRole,
        layer_index: int | None = None,
        expert_index: int | None = None,
        expert_scope: ExpertScope = ExpertScope.NONE,
        shard_dim: int | None = None,
        allow_quantization: bool = True,
    ) -> nn.Module: ...


# ----------------------------------------------------------------- modules
class QuantizedLinearBase(nn.Module):
    """Shape bookkeeping, optional fp32 bias and device dispatch."""

    is_quantized = True  # loader flag: packed buffers keep their checkpoint dtype
    quant_scheme: str

    def __init__(self, in_features: int, out_features: int, bias: bool) -> None:
        super().__init__()
        if in_features < 1 or out_features < 1:
            raise ValueError("quantized linear dimensions must be positive")
        self.in_features = in_features
        self.out_features = out_features
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)

    def dequantize(self) -> torch.Tensor:  # pragma: no cover - abstract
        raise NotImplementedError

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {"bias": CheckpointMemberLayout(column_dim=0, row_dim=None)}

    def _add_local_bias(self) -> bool:
        return not bool(getattr(self, "_kairyu_row_parallel_omit_bias", False))

    def forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        weight = self.dequantize().to(x.dtype)
        bias = self.bias if self._add_local_bias() else None
        return nn.functional.linear(x, weight, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type == "cuda":
            return self.forward_fused(x)
        return self.forward_reference(x)

    def forward_fused(self, x: torch.Tensor) -> torch.Tensor:
        """Device dispatch to the bound HIP kernel; never dequantizes."""

        bound = getattr(self, "_fused_forward", None)
        if bound is not None:
            return bound(x, self, add_bias=self._add_local_bias())
        from kairyu_amd.kernels.quant_gemm_hip import linear_forward

        return linear_forward(x, self, add_bias=self._add_local_bias())


class Fp8Linear(QuantizedLinearBase):
    """FP8 e4m3 weights with a per-channel ``[out, 1]`` or per-tensor ``(1,)`` scale."""

    quant_scheme = "fp8"

    def __init__(
        self, in_features: int, out_features: int, bias: bool, activation_dynamic: bool = True
    ) -> None:
        super().__init__(in_features, out_features, bias)
        self.activation_dynamic = activation_dynamic
        self.register_buffer(
            "weight", torch.zeros(out_features, in_features, dtype=torch.float8_e4m3fn)
        )
        self.register_buffer("weight_scale", torch.ones(out_features, 1))
        if not activation_dynamic:
            self.register_buffer("input_scale", torch.ones(()))

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        # A per-tensor checkpoint ships a (1,) scale; adopt whichever scale
        # shape the checkpoint carries so both variants load.
        incoming = state_dict.get(prefix + "weight_scale")
        if incoming is not None and incoming.shape != self.weight_scale.shape:
            self.register_buffer("weight_scale", torch.empty_like(incoming))
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    def dequantize(self) -> torch.Tensor:
        return fp8.dequantize_fp8(self.weight, self.weight_scale)

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {
            **super().checkpoint_member_layouts(),
            "weight": CheckpointMemberLayout(column_dim=0, row_dim=1),
            "weight_scale": CheckpointMemberLayout(column_dim=0, row_dim=None),
            "input_scale": CheckpointMemberLayout(column_dim=None, row_dim=None),
        }

    def _finish(self, out: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        if self.bias is not None and self._add_local_bias():
            out = out + self.bias
        return out.to(dtype)

    def forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        input_scale = None if self.activation_dynamic else self.input_scale
        x_q, x_scale = fp8.quantize_fp8_activation(x.to(torch.float32), scale=input_scale)
        out = fp8.fp8_w8a8_matmul(x_q, x_scale, self.weight, self.weight_scale)
        return self._finish(out, x.dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Honor a row-parallel owner that supplies a global per-token scale."""

        comm = getattr(self, "_row_parallel_comm", None)
        if comm is not None and self.activation_dynamic:
            local_amax = self.activation_amax(x).contiguous()
            global_amax = comm.tensor_all_reduce_max(local_amax)
            scale = (global_amax / fp8.FP8_MAX).clamp(min=1e-12)
            return self.forward_with_activation_scale(x, scale)
        return super().forward(x)

    def activation_amax(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type == "cuda":
            from kairyu_amd.kernels.quant_gemm_hip import fp8_activation_amax

            return fp8_activation_amax(x)
        return x.to(torch.float32).abs().amax(dim=-1, keepdim=True)

    def forward_with_activation_scale(
        self, x: torch.Tensor, activation_scale: torch.Tensor
    ) -> torch.Tensor:
        if not self.activation_dynamic:
            raise ValueError("a global per-token scale requires dynamic FP8 activation")
        activation_scale = activation_scale.to(device=x.device, dtype=torch.float32).clamp(
            min=1e-12
        )
        if x.device.type == "cuda":
            bound = getattr(self, "_fused_forward", None)
            if bound is None:
                from kairyu_amd.kernels.quant_gemm_hip import fp8_linear_forward

                bound = fp8_linear_forward
            return bound(
                x, self, activation_scale=activation_scale, add_bias=self._add_local_bias()
            )
        scaled = (x.to(torch.float32) / activation_scale).clamp(-fp8.FP8_MAX, fp8.FP8_MAX)
        out = fp8.fp8_w8a8_matmul(
            scaled.to(torch.float8_e4m3fn), activation_scale, self.weight, self.weight_scale
        )
        return self._finish(out, x.dtype)


class Int8Linear(QuantizedLinearBase):
    """Per-channel symmetric int8 weights, dynamic per-token int8 activations."""

    quant_scheme = "int8"

    def __init__(self, in_features: int, out_features: int, bias: bool) -> None:
        super().__init__(in_features, out_features, bias)
        self.register_buffer("weight", torch.zeros(out_features, in_features, dtype=torch.int8))
        self.register_buffer("weight_scale", torch.ones(out_features, 1))

    def dequantize(self) -> torch.Tensor:
        return int8.dequantize_int8(self.weight, self.weight_scale)

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {
            **super().checkpoint_member_layouts(),
            "weight": CheckpointMemberLayout(column_dim=0, row_dim=1),
            "weight_scale": CheckpointMemberLayout(column_dim=0, row_dim=None),
        }

    def forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        x_q, x_scale = int8.quantize_int8_activation(x.to(torch.float32))
        out = int8.int8_w8a8_matmul(x_q, x_scale, self.weight, self.weight_scale)
        if self.bias is not None and self._add_local_bias():
            out = out + self.bias
        return out.to(x.dtype)


def _resolve_group_size(group_size: int, in_features: int) -> int:
    """``group_size <= 0`` (checkpoint ``-1``) means one group over all inputs."""

    return in_features if group_size <= 0 else group_size


_PACKED = CheckpointMemberLayout(column_dim=1, row_dim=0)


class AwqLinear(QuantizedLinearBase):
    quant_scheme = "awq"

    def __init__(
        self, in_features: int, out_features: int, bias: bool, group_size: int = 128
    ) -> None:
        super().__init__(in_features, out_features, bias)
        group_size = _resolve_group_size(group_size, in_features)
        if out_features % 8:
            raise ValueError("AWQ out_features must be divisible by 8")
        if in_features % group_size:
            raise ValueError("AWQ in_features must be divisible by group_size")
        self.group_size = group_size
        groups = in_features // group_size
        self.register_buffer(
            "qweight", torch.zeros(in_features, out_features // 8, dtype=torch.int32)
        )
        self.register_buffer("qzeros", torch.zeros(groups, out_features // 8, dtype=torch.int32))
        self.register_buffer("scales", torch.ones(groups, out_features, dtype=torch.float16))

    def dequantize(self) -> torch.Tensor:
        return awq.dequantize_awq(self.qweight, self.qzeros, self.scales, self.group_size)

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {
            **super().checkpoint_member_layouts(),
            "qweight": _PACKED,
            "qzeros": _PACKED,
            "scales": _PACKED,
        }


class GptqLinear(QuantizedLinearBase):
    quant_scheme = "gptq"

    def __init__(
        self, in_features: int, out_features: int, bias: bool, group_size: int = 128
    ) -> None:
        super().__init__(in_features, out_features, bias)
        group_size = _resolve_group_size(group_size, in_features)
        if in_features % 8 or out_features % 8:
            raise ValueError("GPTQ in_features and out_features must be divisible by 8")
        self.group_size = group_size
        groups = -(-in_features // group_size)
        self.register_buffer(
            "qweight", torch.zeros(in_features // 8, out_features, dtype=torch.int32)
        )
        self.register_buffer("qzeros", torch.zeros(groups, out_features // 8, dtype=torch.int32))
        self.register_buffer("scales", torch.ones(groups, out_features, dtype=torch.float16))
        self.register_buffer("g_idx", torch.zeros(in_features, dtype=torch.int32))

    def dequantize(self) -> torch.Tensor:
        return gptq.dequantize_gptq(
            self.qweight, self.qzeros, self.scales, self.g_idx, self.group_size
        )

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {
            **super().checkpoint_member_layouts(),
            "qweight": _PACKED,
            "qzeros": _PACKED,
            "scales": _PACKED,
            "g_idx": CheckpointMemberLayout(column_dim=None, row_dim=0),
        }


class BlockFp8Linear(QuantizedLinearBase):
    """128x128 block-scaled FP8 weights with dynamic 1x128 activation blocks.

    Buffers follow the DeepSeek-style checkpoint names: ``weight`` e4m3
    ``[out, in]`` and ``weight_scale_inv`` fp32 ``[ceil(out/128), ceil(in/128)]``.
    """

    quant_scheme = "fp8_block"

    def __init__(self, in_features: int, out_features: int, bias: bool) -> None:
        super().__init__(in_features, out_features, bias)
        self.register_buffer(
            "weight", torch.zeros(out_features, in_features, dtype=torch.float8_e4m3fn)
        )
        self.register_buffer(
            "weight_scale_inv",
            torch.ones(-(-out_features // block_fp8.BLOCK), -(-in_features // block_fp8.BLOCK)),
        )

    def dequantize(self) -> torch.Tensor:
        return block_fp8.dequantize_block_fp8(self.weight, self.weight_scale_inv)

    def checkpoint_member_layouts(self) -> dict[str, CheckpointMemberLayout]:
        return {
            **super().checkpoint_member_layouts(),
            "weight": CheckpointMemberLayout(column_dim=0, row_dim=1),
            "weight_scale_inv": CheckpointMemberLayout(column_dim=0, row_dim=1),
        }

    def forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        x_q, x_scale = block_fp8.quantize_block_fp8_activation(x.to(torch.float32))
        out = block_fp8.block_fp8_matmul(x_q, x_scale, self.weight, self.weight_scale_inv)
        if self.bias is not None and self._add_local_bias():
            out = out + self.bias
        return out.to(x.dtype)


# ------------------------------------------------------------ construction
def _construct_linear(
    quant: QuantConfig, in_features: int, out_features: int, bias: bool
) -> nn.Module:
    method = quant.method
    if method is QuantMethod.NONE:
        return nn.Linear(in_features, out_features, bias=bias)
    if method is QuantMethod.FP8:
        return Fp8Linear(
            in_features, out_features, bias, activation_dynamic=quant.activation_dynamic is not False
        )
    if method is QuantMethod.INT8:
        return Int8Linear(in_features, out_features, bias)
    if method is QuantMethod.AWQ:
        return AwqLinear(in_features, out_features, bias, group_size=quant.group_size or 128)
    if method is QuantMethod.GPTQ:
        return GptqLinear(in_features, out_features, bias, group_size=quant.group_size or 128)
    if method is QuantMethod.FP8_BLOCK:
        return BlockFp8Linear(in_features, out_features, bias)
    raise ValueError(f"no QuantizedLinear for {method}")  # pragma: no cover


def _ignore_matches(pattern: str, name: str) -> bool:
    if pattern.startswith("re:"):
        try:
            return re.fullmatch(pattern[3:], name) is not None
        except re.error as error:
            raise ValueError(f"invalid quantization ignore pattern {pattern!r}") from error
    return name == pattern or name.startswith(pattern + ".")


_DENSE_ROLES = frozenset({LinearRole.MOE_ROUTER, LinearRole.DRAFT_FUSION, LinearRole.OUTPUT_HEAD})


def default_linear_selection(quant: QuantConfig, context: LinearBuildContext) -> LinearSelection:
    """Architectural exclusion, then checkpoint ignores, then dense-by-role.

    Routers, output heads and draft fusion stay dense: their near-ties are
    unusually sensitive to quantization error (linear.py:854-896).
    """

    dense = QuantConfig(method=QuantMethod.NONE)
    if not context.allow_quantization:
        return LinearSelection(dense, None, "architectural-exclusion")
    for pattern in quant.ignored_layers:
        if _ignore_matches(pattern, context.qualified_name):
            return LinearSelection(dense, None, f"checkpoint-ignore:{pattern}")
    if context.role in _DENSE_ROLES:
        return LinearSelection(dense, None, f"default-dense-role:{context.role.value}")
    return LinearSelection(quant, None, "checkpoint-format")


def _context_description(context: LinearBuildContext) -> str:
    tp = context.tensor_parallel
    return (
        f"name={context.qualified_name!r}, scope={context.model_scope.value}, "
        f"role={context.role.value}, device={context.device}, dtype={context.dtype}, "
        f"tp={tp.mode.value}:{tp.rank}/{tp.world_size}:dim={tp.shard_dim}, "
        f"local={tp.local_in_features}x{tp.local_out_features}, "
        f"global={tp.global_in_features}x{tp.global_out_features}, "
        f"capabilities={context.capabilities.source}"
    )


def _bind_fused_forward(module: nn.Module, selection: LinearSelection, device: torch.device) -> None:
    if device.type != "cuda" or selection.quantization.method is QuantMethod.NONE:
        return
    from kairyu_amd.kernels import quant_gemm_hip as hip

    table = {
        (LinearKernel.HIP_FP8_W8A8, QuantMethod.FP8): hip.fp8_linear_forward,
        (LinearKernel.HIP_INT8_W8A8, QuantMethod.INT8): hip.int8_linear_forward,
        (LinearKernel.HIP_W4A16, QuantMethod.AWQ): hip.awq_linear_forward,
        (LinearKernel.HIP_W4A16, QuantMethod.GPTQ): hip.gptq_linear_forward,
        (LinearKernel.HIP_FP8_BLOCK, QuantMethod.FP8_BLOCK): hip.block_fp8_linear_forward,
    }
    key = (selection.kernel, selection.quantization.method)
    if key not in table:
        raise RuntimeError(
            "no bound forward implementation for "
            f"{selection.kernel.value}/{selection.quantization.method.value}"
        )
    module._fused_forward = table[key]


class ContextualLinearFactory:
    """Projection factory with target device, dtype and TP placement bound once.

    Unsupported quantized selections fail at construction; an implicit dense
    fallback would misread packed checkpoint tensors and is forbidden.
    """

    def __init__(
        self,
        quant: QuantConfig,
        *,
        device: str | torch.device = "cpu",
        dtype: torch.dtype = torch.float32,
        tensor_parallel_size: int = 1,
        tensor_parallel_rank: int = 0,
        capabilities: LinearKernelCapabilities | None = None,
        selection_policy: LinearSelectionPolicy | None = None,
    ) -> None:
        if not isinstance(dtype, torch.dtype):
            raise TypeError("linear target dtype must be a torch.dtype")
        if tensor_parallel_size < 1:
            raise ValueError("tensor-parallel world_size must be positive")
        if not 0 <= tensor_parallel_rank < tensor_parallel_size:
            raise ValueError(
                f"tensor-parallel rank {tensor_parallel_rank} is outside "
                f"world_size {tensor_parallel_size}"
            )
        self._quant = quant
        self._device = torch.device(device)
        self._dtype = dtype
        self._world_size = tensor_parallel_size
        self._rank = tensor_parallel_rank
        self._capabilities = capabilities or LinearKernelCapabilities.for_device(self._device)
        self._selection_policy = selection_policy or default_linear_selection

    def _placement(self, in_features: int, out_features: int, shard_dim: int | None):
        modes = {None: TensorParallelMode.REPLICATED, 0: TensorParallelMode.COLUMN, 1: TensorParallelMode.ROW}
        if shard_dim not in modes:
            raise ValueError("tensor-parallel shard_dim must be 0, 1, or None")
        mode = modes[shard_dim]
        scale_in = self._world_size if mode is TensorParallelMode.ROW else 1
        scale_out = self._world_size if mode is TensorParallelMode.COLUMN else 1
        return TensorParallelPlacement(
            mode=mode,
            world_size=self._world_size,
            rank=self._rank,
            shard_dim=shard_dim,
            global_in_features=in_features * scale_in,
            global_out_features=out_features * scale_out,
            local_in_features=in_features,
            local_out_features=out_features,
        )

    def __call__(
        self,
        in_features: int,
        out_features: int,
        bias: bool,
        *,
        qualified_name: str | None = None,
        model_scope: ModelScope = ModelScope.TARGET,
        role: LinearRole | None = None,
        layer_index: int | None = None,
        expert_index: int | None = None,
        expert_scope: ExpertScope = ExpertScope.NONE,
        shard_dim: int | None = None,
        allow_quantization: bool = True,
    ) -> nn.Module:
        if qualified_name is None and role is None:
            # legacy three-argument contract: no identity, no selection metadata
            return _construct_linear(self._quant, in_features, out_features, bias)
        if qualified_name is None or role is None:
            raise TypeError("contextual linear construction requires both qualified_name and role")
        context = LinearBuildContext(
            qualified_name=qualified_name,
            model_scope=model_scope,
            role=role,
            device=self._device,
            dtype=self._dtype,
            tensor_parallel=self._placement(in_features, out_features, shard_dim),
            capabilities=self._capabilities,
            layer_index=layer_index,
            expert_index=expert_index,
            expert_scope=expert_scope,
            allow_quantization=allow_quantization,
        )
        selected = self._selection_policy(self._quant, context)
        if not isinstance(selected, LinearSelection):
            raise TypeError(
                f"linear selection policy must return LinearSelection for {qualified_name!r}"
            )
        method = selected.quantization.method
        if not allow_quantization and method is not QuantMethod.NONE:
            raise ValueError(
                f"linear {qualified_name!r} ({role.value}) excludes quantization, "
                f"but policy selected {method.value}"
            )
        kernel = selected.kernel or self._capabilities.preferred_kernel(method)
        if kernel is None:
            raise RuntimeError(
                f"no production kernel for {method.value}; {_context_description(context)}"
            )
        if kernel not in self._capabilities.available_kernels or method not in _KERNEL_METHODS[kernel]:
            raise RuntimeError(
                f"kernel {kernel.value} cannot serve {method.value}; {_context_description(context)}"
            )
        on_device = self._device.type == "cuda"
        host_kernels = {LinearKernel.TORCH_DENSE, LinearKernel.CPU_REFERENCE}
        if (on_device and kernel is LinearKernel.CPU_REFERENCE) or (
            not on_device and kernel not in host_kernels
        ):
            raise RuntimeError(
                f"kernel {kernel.value} is incompatible with target {self._device.type}; "
                f"{_context_description(context)}"
            )
        if on_device and method is not QuantMethod.NONE and self._dtype not in (
            torch.float16,
            torch.bfloat16,
        ):
            raise ValueError(
                "quantized device compute requires float16 or bfloat16; "
                f"{_context_description(context)}"
            )
        resolved = LinearSelection(
            selected.quantization, kernel, selected.reason, selected.observe_activation_saturation
        )
        module = _construct_linear(selected.quantization, in_features, out_features, bias)
        _bind_fused_forward(module, resolved, self._device)
        module.linear_context = context
        module.linear_selection = resolved
        return module


def linear_factory(
    quant: QuantConfig,
    *,
    device: str | torch.device = "cpu",
    dtype: torch.dtype = torch.float32,
    tensor_parallel_size: int = 1,
    tensor_parallel_rank: int = 0,
    capabilities: LinearKernelCapabilities | None = None,
    selection_policy: LinearSelectionPolicy | None = None,
) -> LinearFactory:
    return ContextualLinearFactory(
        quant,
        device=device,
        dtype=dtype,
        tensor_parallel_size=tensor_parallel_size,
        tensor_parallel_rank=tensor_parallel_rank,
        capabilities=capabilities,
        selection_policy=selection_policy,
    )


def make_linear(
    factory: LinearFactory | None,
    in_features: int,
    out_features: int,
    bias: bool,
    *,
    qualified_name: str,
    model_scope: ModelScope = ModelScope.TARGET,
    role: LinearRole,
    layer_index: int | None = None,
    expert_index: int | None = None,
    expert_scope: ExpertScope = ExpertScope.NONE,
    shard_dim: int | None = None,
    allow_quantization: bool = True,
) -> nn.Module:
    """Construct one projection; ``factory=None`` keeps a plain ``nn.Linear``."""

    if factory is None:
        return nn.Linear(in_features, out_features, bias=bias)
    kwargs = {
        "qualified_name": qualified_name,
        "model_scope": model_scope,
        "role": role,
        "layer_index": layer_index,
        "expert_index": expert_index,
        "expert_scope": expert_scope,
        "shard_dim": shard_dim,
        "allow_quantization": allow_quantization,
    }
    if isinstance(factory, ContextualLinearFactory):
        return factory(in_features, out_features, bias, **kwargs)
    try:
        inspect.signature(factory).bind(in_features, out_features, bias, **kwargs)
    except (TypeError, ValueError):
        # legacy three-argument factories; binding (not calling) decides, so an
        # error raised inside the factory is never masked
        return factory(in_features, out_features, bias)
    return factory(in_features, out_features, bias, **kwargs)
