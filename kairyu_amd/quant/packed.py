"""One launch for several quantized projections of the same input.

The reference packs plain dense Q/K/V (and NVFP4) projections into one
output-row-contiguous weight so that one GEMM replaces three
(``kairyu/models/packed_linear.py:30-218``, ``DenseLinearPack``; used by
``kairyu/models/attention.py:105-160``).  ``QuantLinearPack`` does the same
for this package's quantized formats:

* FP8 / INT8 W8A8 (``Fp8Linear``, ``Int8Linear``): the ``[N, K]`` weights are
  concatenated once into one allocation and every projection's ``weight``
  buffer becomes a row view of it, exactly as ``DenseLinearPack`` re-points
  its parameters, so ``state_dict`` keeps the checkpoint names and values.  One
  per-token activation quantization and one GEMM serve all projections.
* AWQ / GPTQ W4A16 (``AwqLinear``, ``GptqLinear``): ``N`` is the packed minor
  dimension of those checkpoints, so their buffers stay untouched; the pack
  keeps derived operands (the projections' columns side by side, tiled as one
  weight with its zeros and fp16 scales), rebuilt when
  a source tensor's version changes, as the single-module derived operands
  are.  GPTQ projections pack when they share one ``g_idx`` (uniform groups,
  or one act-order permutation, so one activation gather serves all).

``swiglu(x)`` of a (gate, up) pack returns ``silu(gate(x)) * up(x)``, the
reference MLP's activation (``kairyu/models/layers.py:243-244``), with
torch's fp16 / bf16 roundings; for W4A16 in one call whose decode GEMV (M <=
16) or prefill GEMM (M > 64) applies SwiGLU in its epilogue (gate and up
16-column blocks interleaved in a derived tiled operand), for W8A8 in one
call whose prefill tile engine or decode GEMM (M <= 16) applies it in its
epilogue (gate rows [n0, n0 + 128) paired with up rows [I + n0, ...) of the
packed weight, or 8 gate and 8 up rows per decode workgroup; no second
copy).

``create`` returns ``None`` for anything it cannot pack exactly (mixed
formats, in-features, devices, biases, group sizes, static input scales,
``g_idx``; hooked or re-bound modules; ``N`` not a multiple of 16 for the
W4A16 tiles).  A call returns one output view per projection, each equal to
what that projection alone computes up to the fp32 accumulation order of the
kernel the packed shape selects (INT8: bit-identical).  On a CPU tensor each
projection runs its own reference forward.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import nn

from .linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear

_SCHEMES = {Fp8Linear: "fp8", Int8Linear: "int8", AwqLinear: "awq", GptqLinear: "gptq"}


def _plain(module: nn.Module) -> bool:
    return not (
        "forward" in module.__dict__
        or module._forward_hooks
        or module._forward_pre_hooks
        or module._backward_hooks
    )


def _key(tensors) -> tuple:
    return tuple((id(t), t._version) for t in tensors)


class QuantLinearPack:
    """Several same-format quantized projections executed as one."""

    __slots__ = ("_projections", "_scheme", "_out_features", "_weight", "_derived", "_derived_key",
                 "_swiglu", "_swiglu_key")

    def __init__(self, projections: tuple[nn.Module, ...], scheme: str,
                 weight: torch.Tensor | None) -> None:
        self._projections = projections
        self._scheme = scheme
        self._out_features = tuple(int(m.out_features) for m in projections)
        self._weight = weight
        self._derived: dict[str, torch.Tensor | int | None] | None = None
        self._derived_key: tuple | None = None
        self._swiglu: dict | None = None
        self._swiglu_key: tuple | None = None

    # ------------------------------------------------------------ creation
    @classmethod
    def create(cls, projections: Sequence[nn.Module]) -> QuantLinearPack | None:
        """Pack compatible projections, otherwise return ``None``."""

        mods = tuple(projections)
        if len(mods) < 2:
            return None
        kind = type(mods[0])
        scheme = _SCHEMES.get(kind)
        if scheme is None or any(type(m) is not kind for m in mods) or not all(map(_plain, mods)):
            return None
        first = mods[0]
        payload = list(first.buffers(recurse=False))
        if not payload or payload[0].device.type == "meta":
            return None
        device = payload[0].device
        has_bias = first.bias is not None
        for m in mods:
            if m.in_features != first.in_features or (m.bias is not None) != has_bias:
                return None
            if any(t.device != device for t in m.buffers(recurse=False)):
                return None
            if has_bias and (m.bias.device != device or m.bias.dtype != first.bias.dtype):
                return None
            if getattr(m, "_kairyu_row_parallel_omit_bias", False) != getattr(
                    first, "_kairyu_row_parallel_omit_bias", False):
                return None
        from kairyu_amd.kernels.quant_gemm_hip import _validate_layout

        try:
            for m in mods:
                _validate_layout(m, scheme)
        except (ValueError, RuntimeError):
            return None

        weight = None
        if scheme in ("fp8", "int8"):
            if scheme == "fp8":
                if any(m.activation_dynamic != first.activation_dynamic for m in mods):
                    return None
                if not first.activation_dynamic and any(
                        not torch.equal(m.input_scale, first.input_scale) for m in mods):
                    return None
            if any(not m.weight.is_contiguous() for m in mods):
                return None
            with torch.no_grad():
                weight = torch.cat([m.weight.detach() for m in mods], dim=0).contiguous()
            row = 0
            for m in mods:
                m._buffers["weight"] = weight.narrow(0, row, m.out_features)
                row += m.out_features
        else:
            if any(m.group_size != first.group_size or m.out_features % 16 != 0 for m in mods):
                return None
            if scheme == "awq" and (first.in_features % 8 != 0 or first.group_size % 8 != 0):
                return None
            if scheme == "gptq":
                if any(not torch.equal(m.g_idx, first.g_idx) for m in mods):
                    return None
                from kairyu_amd.kernels.quant_gemm_hip import GIDX_PER_K, gptq_group_mode

                if device.type == "cuda" and gptq_group_mode(
                        first.g_idx, first.in_features, first.group_size, device)[0] == GIDX_PER_K:
                    return None
        return cls(mods, scheme, weight)

    # --------------------------------------------------------- bookkeeping
    @property
    def out_features(self) -> tuple[int, ...]:
        return self._out_features

    @property
    def projections(self) -> tuple[nn.Module, ...]:
        return self._projections

    def matches(self, projections: Sequence[nn.Module]) -> bool:
        """Whether the owner's canonical modules are still the packed ones."""

        return len(projections) == len(self._projections) and all(
            a is b for a, b in zip(projections, self._projections, strict=True))

    def is_current(self) -> bool:
        """Whether the canonical modules still describe this pack: same
        shapes, no re-bound forwards or hooks, and (W8A8) every ``weight``
        still the row view of the packed allocation the pack was built with."""

        for m, n in zip(self._projections, self._out_features, strict=True):
            if not _plain(m) or m.out_features != n:
                return False
        if self._weight is None:
            return True
        base = self._weight.untyped_storage().data_ptr()
        offset = self._weight.storage_offset()
        k = self._projections[0].in_features
        row = 0
        for m, n in zip(self._projections, self._out_features, strict=True):
            w = m.weight
            if (tuple(w.shape) != (n, k) or w.stride() != (k, 1)
                    or w.untyped_storage().data_ptr() != base
                    or w.storage_offset() != offset + row * k):
                return False
            row += n
        return True

    # ------------------------------------------------------ derived operands
    def _sources(self) -> list[torch.Tensor]:
        out = []
        for m in self._projections:
            if self._scheme in ("fp8", "int8"):
                out.append(m.weight_scale)
                if self._scheme == "fp8" and not m.activation_dynamic:
                    out.append(m.input_scale)
            elif self._scheme == "awq":
                out += [m.qweight, m.qzeros, m.scales]
            else:
                out += [m.qweight, m.qzeros, m.scales, m.g_idx]
            if m.bias is not None:
                out.append(m.bias)
        return out

    def _operands(self, device: torch.device) -> dict:
        key = (_key(self._sources()), str(device))
        if self._derived is not None and self._derived_key == key:
            return self._derived
        from kairyu_amd.kernels import quant_gemm_hip as hip

        mods = self._projections
        d: dict = {"bias": None}
        with torch.no_grad():
            if mods[0].bias is not None:
                d["bias"] = torch.cat([m.bias.detach().reshape(-1) for m in mods]).contiguous()
            if self._scheme in ("fp8", "int8"):
                first = mods[0]
                if self._scheme == "fp8" and not first.activation_dynamic and any(
                        not torch.equal(m.input_scale, first.input_scale) for m in mods):
                    raise RuntimeError("packed FP8 projections need one static input_scale")
                # per-channel fp32 scales (a per-tensor FP8 scale repeats per row)
                d["weight_scale"] = torch.cat([
                    hip._f32(m.weight_scale).expand(m.out_features) if m.weight_scale.numel() == 1
                    else hip._f32(m.weight_scale) for m in mods]).contiguous()
            elif self._scheme == "awq":
                # the packed columns tiled as one weight (tiles and their
                # scale/zero table)
                zeros = torch.cat([hip.awq_natural_zeros(m.qzeros, m.out_features, device)
                                   for m in mods], dim=1).contiguous()
                d["scales"] = torch.cat([m.scales for m in mods], dim=1).contiguous()
                d["perm"], d["mode"] = None, hip.GIDX_UNIFORM
                d["tiled"] = hip.tile_operand(
                    torch.cat([m.qweight for m in mods], dim=1).contiguous(), 0, None, zeros, 0,
                    d["scales"], sum(self._out_features), mods[0].in_features, mods[0].group_size,
                    device)
                if d["tiled"] is None:
                    raise RuntimeError("AWQ pack requires tileable projections")
                for m in mods:  # the pack holds the only tiled copy
                    m.__dict__.pop("_kq_awq_operands", None)
            else:
                first = mods[0]
                if any(not torch.equal(m.g_idx, first.g_idx) for m in mods[1:]):
                    # one activation gather serves every projection
                    raise RuntimeError("packed GPTQ projections need one g_idx")
                ops = [hip._gptq_operands(m, device) for m in mods]
                if any(mode == hip.GIDX_PER_K for mode, _, _ in ops):
                    raise RuntimeError("GPTQ pack requires uniform or act-order groups")
                if any(mode != ops[0][0] for mode, _, _ in ops):
                    raise RuntimeError("packed GPTQ projections need one group mode")
                zeros = torch.cat([m.qzeros for m in mods], dim=1).contiguous()
                d["scales"] = torch.cat([m.scales for m in mods], dim=1).contiguous()
                d["perm"], d["mode"] = ops[0][2], ops[0][0]
                d["tiled"] = hip.tile_operand(
                    torch.cat([m.qweight for m in mods], dim=1).contiguous(), 1, d["perm"],
                    zeros, 1, d["scales"], sum(self._out_features), mods[0].in_features,
                    mods[0].group_size, device)
                for m in mods:
                    m.__dict__.pop("_kq_gptq_operands", None)
        self._derived, self._derived_key = d, key
        return d

    # ------------------------------------------------------------- forward
    def __call__(self, hidden: torch.Tensor) -> tuple[torch.Tensor, ...]:
        if not self.is_current():
            raise RuntimeError("canonical projection buffers no longer match the packed storage")
        if hidden.device.type != "cuda":
            return tuple(m(hidden) for m in self._projections)
        out = self._packed(hidden)
        lead = hidden.shape[:-1]
        return tuple(part.reshape(*lead, part.shape[-1]) for part in out.split(self._out_features, -1))

    def swiglu(self, hidden: torch.Tensor) -> torch.Tensor:
        """``silu(gate(x)) * up(x)`` of a (gate, up) pack, as the reference's
        MLP computes it (``kairyu/models/layers.py:243-244``) with torch's
        roundings on fp16/bf16 tensors.  W4A16 packs run one call whose decode
        GEMV or prefill GEMM applies SwiGLU in its epilogue (gate and up
        columns interleaved by 16 in a derived tiled operand,
        ``kq_w4a16_tiled_swiglu_gemm``);
        W8A8 packs run ``kq_w8a8_*_swiglu_linear`` (SwiGLU in the tile
        engine's epilogue for prefill shapes, in the decode GEMM's for
        M <= 16)."""

        if len(self._projections) != 2 or self._out_features[0] != self._out_features[1]:
            raise ValueError("swiglu needs a (gate, up) pack of equal widths")
        if not self.is_current():
            raise RuntimeError("canonical projection buffers no longer match the packed storage")
        gate, up = self._projections
        if hidden.device.type != "cuda":
            return nn.functional.silu(gate(hidden)) * up(hidden)
        from kairyu_amd import _native
        from kairyu_amd.kernels import quant_gemm_hip as hip

        width = self._out_features[0]
        lead = hidden.shape[:-1]
        stream = _native.stream_handle(hidden.device)
        if self._scheme in ("fp8", "int8"):
            return self._w8a8_swiglu(hidden, width).reshape(*lead, width)
        flat, _ = hip._prepare(hidden, gate, self._scheme, allocate_output=False)
        hip._validate_layout(up, self._scheme)
        d = self._swiglu_operands(hidden.device)
        m_rows, k = flat.shape
        act = torch.empty((m_rows, width), device=hidden.device, dtype=hidden.dtype)
        bias = d["bias"] if gate._add_local_bias() else None
        ws = hip._workspace(hidden.device, int(_native.library().kq_w4a16_swiglu_workspace_size(
            m_rows, width, k, d["mode"])))
        _native.call(
            "kq_w4a16_tiled_swiglu_gemm", flat.data_ptr(), _native.dtype_code(flat.dtype),
            d["tiled"].tiles.data_ptr(), _native.ptr(d["tiled"].zeros), d["tiled"].zero_offset,
            d["scales"].data_ptr(), _native.ptr(d["perm"]), _native.ptr(bias),
            _native.dtype_code(None if bias is None else bias.dtype), act.data_ptr(), m_rows, width,
            k, gate.group_size, ws.data_ptr(), ws.numel(), stream,
        )
        return act.reshape(*lead, width)

    def _w8a8_swiglu(self, hidden: torch.Tensor, width: int) -> torch.Tensor:
        """One kq_w8a8_*_swiglu_linear call on the packed [gate; up] weight:
        SwiGLU in the tile engine's epilogue for prefill shapes and in the
        decode GEMM's for M <= 16, the packed GEMM and the elementwise pass
        otherwise (the same bits either way)."""

        from kairyu_amd import _native
        from kairyu_amd.kernels import quant_gemm_hip as hip

        gate = self._projections[0]
        flat, _ = hip._prepare(hidden, gate, self._scheme, allocate_output=False)
        hip._validate_layout(self._projections[1], self._scheme)
        d = self._operands(hidden.device)
        m_rows, k = flat.shape
        act = torch.empty((m_rows, width), device=hidden.device, dtype=hidden.dtype)
        bias = d["bias"] if gate._add_local_bias() else None
        bias_args = (_native.ptr(bias), _native.dtype_code(None if bias is None else bias.dtype))
        ws = hip._workspace(hidden.device, int(_native.library().kq_w8a8_swiglu_workspace_size(m_rows, width, k)))
        stream = _native.stream_handle(hidden.device)
        if self._scheme == "fp8":
            mode, source = (0, None) if gate.activation_dynamic else (1, hip._f32(gate.input_scale))
            _native.call("kq_w8a8_fp8_swiglu_linear", flat.data_ptr(), _native.dtype_code(flat.dtype),
                         flat.stride(0), _native.ptr(source), mode, self._weight.data_ptr(),
                         d["weight_scale"].data_ptr(), 1, *bias_args, act.data_ptr(), m_rows, width, k,
                         ws.data_ptr(), ws.numel(), stream)
        else:
            _native.call("kq_w8a8_i8_swiglu_linear", flat.data_ptr(), _native.dtype_code(flat.dtype),
                         flat.stride(0), self._weight.data_ptr(), d["weight_scale"].data_ptr(), *bias_args,
                         act.data_ptr(), m_rows, width, k, ws.data_ptr(), ws.numel(), stream)
        return act

    def _swiglu_operands(self, device: torch.device) -> dict:
        """The (gate, up) pair tiled as one weight whose 16-column blocks of
        gate and up alternate (the SwiGLU epilogue holds both halves of a
        pair), with its scales, zeros and bias in the same column order."""

        key = (_key(self._sources()), str(device))
        if self._swiglu is not None and self._swiglu_key == key:
            return self._swiglu
        from kairyu_amd.kernels import quant_gemm_hip as hip

        hip._refuse_under_capture(self._scheme.upper())
        gate, up = self._projections

        def mix(a: torch.Tensor, b: torch.Tensor, block: int) -> torch.Tensor:
            # column blocks of a and b alternating: [a0, b0, a1, b1, ...]
            a2, b2 = a.reshape(a.shape[0], -1, block), b.reshape(b.shape[0], -1, block)
            return torch.stack([a2, b2], dim=2).reshape(a.shape[0], -1).contiguous()

        d: dict = {"bias": None}
        with torch.no_grad():
            if gate.bias is not None:
                d["bias"] = mix(gate.bias.detach().reshape(1, -1), up.bias.detach().reshape(1, -1), 16).reshape(-1)
            d["scales"] = mix(gate.scales, up.scales, 16)
            if self._scheme == "awq":
                zeros = mix(hip.awq_natural_zeros(gate.qzeros, gate.out_features, device),
                            hip.awq_natural_zeros(up.qzeros, up.out_features, device), 2)
                qweight, fmt, zoff, d["perm"], d["mode"] = mix(gate.qweight, up.qweight, 2), 0, 0, None, hip.GIDX_UNIFORM
            else:
                if not torch.equal(up.g_idx, gate.g_idx):
                    # one activation gather serves both halves
                    raise RuntimeError("packed GPTQ projections need one g_idx")
                # the group mode and permutation alone: tiling gate on its own
                # here would cache a second tiled copy of its weights
                mode, perm = hip.gptq_group_mode(gate.g_idx, gate.in_features, gate.group_size, device)
                if mode == hip.GIDX_PER_K:
                    raise RuntimeError("GPTQ swiglu pack requires uniform or act-order groups")
                zeros = mix(gate.qzeros, up.qzeros, 2)
                qweight, fmt, zoff, d["perm"], d["mode"] = mix(gate.qweight, up.qweight, 16), 1, 1, perm, mode
            d["tiled"] = hip.tile_operand(qweight, fmt, d["perm"], zeros, zoff, d["scales"],
                                          2 * gate.out_features, gate.in_features, gate.group_size, device)
            if d["tiled"] is None:
                raise RuntimeError("swiglu pack requires tileable projections")
            for m in (gate, up):  # the pack holds the only tiled copies
                m.__dict__.pop("_kq_gptq_operands", None)
                m.__dict__.pop("_kq_awq_operands", None)
        self._swiglu, self._swiglu_key = d, key
        return d

    def _packed(self, hidden: torch.Tensor) -> torch.Tensor:
        """The projections' outputs side by side, [rows, sum(out_features)]."""

        from kairyu_amd import _native
        from kairyu_amd.kernels import quant_gemm_hip as hip

        first = self._projections[0]
        flat, _ = hip._prepare(hidden, first, self._scheme, allocate_output=False)
        for m in self._projections[1:]:
            hip._validate_layout(m, self._scheme)
        d = self._operands(hidden.device)
        m_rows, k = flat.shape
        n = sum(self._out_features)
        out = torch.empty((m_rows, n), device=hidden.device, dtype=hidden.dtype)
        bias = d["bias"] if first._add_local_bias() else None
        bias_args = (_native.ptr(bias), _native.dtype_code(None if bias is None else bias.dtype))
        stream = _native.stream_handle(hidden.device)
        if self._scheme in ("fp8", "int8"):
            ws = hip._w8a8_linear_workspace(hidden.device, m_rows, n, k)
            if self._scheme == "fp8":
                mode, source = (0, None) if first.activation_dynamic else (1, hip._f32(first.input_scale))
                _native.call(
                    "kq_w8a8_fp8_linear", flat.data_ptr(), _native.dtype_code(flat.dtype),
                    flat.stride(0), _native.ptr(source), mode, self._weight.data_ptr(),
                    d["weight_scale"].data_ptr(), 1, *bias_args, out.data_ptr(),
                    _native.dtype_code(hidden.dtype), m_rows, n, k, ws.data_ptr(), ws.numel(), stream,
                )
            else:
                _native.call(
                    "kq_w8a8_i8_linear", flat.data_ptr(), _native.dtype_code(flat.dtype),
                    flat.stride(0), self._weight.data_ptr(), d["weight_scale"].data_ptr(),
                    *bias_args, out.data_ptr(), _native.dtype_code(hidden.dtype), None,
                    m_rows, n, k, ws.data_ptr(), ws.numel(), stream,
                )
        else:
            ws = hip._w4_workspace(hidden.device, m_rows, n, k, d["mode"])
            _native.call(
                "kq_w4a16_tiled_gemm", flat.data_ptr(), _native.dtype_code(flat.dtype),
                d["tiled"].tiles.data_ptr(), _native.ptr(d["tiled"].zeros), d["tiled"].zero_offset,
                d["scales"].data_ptr(), _native.ptr(d["perm"]), *bias_args, out.data_ptr(),
                m_rows, n, k, first.group_size, ws.data_ptr(), ws.numel(), stream,
            )
        return out
