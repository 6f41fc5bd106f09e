"""Device forwards of the quantized linear formats on gfx950.

Interface of kairyu/kernels/quant_gemm_gpu.py:409-1024 (``_prepare``,
``_validate_layout``, ``_quantize_activation``, ``fp8_activation_amax``,
``fp8/int8/awq/gptq_linear_forward``, ``linear_forward``).  Each forward
validates fail-closed before launch (RuntimeError for backend / device / dtype
problems, ValueError for shape and packed-layout mismatches), flattens ``x`` to
``[M, K]``, allocates the output in ``x.dtype`` and launches the HIP kernels of
``libkairyu_quant.so`` on torch's current stream.  No path materializes a
floating-point ``[out, in]`` weight and there is no dequantized fallback.
"""

from __future__ import annotations

from typing import NamedTuple

from functools import lru_cache

import torch

from kairyu_amd import _native

REQUIRED_ARCH = "gfx950"


@lru_cache(maxsize=None)
def _arch_of(index: int) -> str:
    return str(torch.cuda.get_device_properties(index).gcnArchName).split(":")[0]


def _device_arch(device: torch.device) -> str:
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _arch_of(index)


def _prepare(x: torch.Tensor, module, scheme: str, *, allocate_output: bool = True):
    try:
        _native.library()
    except RuntimeError as error:
        raise RuntimeError(
            f"{scheme} device execution requires the kairyu_amd HIP library: {error}"
        ) from error
    if not x.is_cuda:
        raise RuntimeError(f"{scheme} fused kernel requires a ROCm device activation")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(
            f"{scheme} fused kernel supports float16/bfloat16 activations, got {x.dtype}"
        )
    arch = _device_arch(x.device)
    if arch != REQUIRED_ARCH:
        raise RuntimeError(
            f"{scheme} fused kernel requires {REQUIRED_ARCH}, got {arch}; "
            "no dequantized GPU fallback exists"
        )
    if x.shape[-1] != module.in_features:
        raise ValueError(f"{scheme} linear expected K={module.in_features}, got {x.shape[-1]}")
    payload = list(module.buffers(recurse=False))
    if module.bias is not None:
        payload.append(module.bias)
    misplaced = [t.device for t in payload if t.device != x.device]
    if misplaced:
        raise RuntimeError(
            f"{scheme} fused kernel requires module payloads on {x.device}; found {misplaced[0]}"
        )
    _validate_layout(module, scheme)
    flat = x.reshape(-1, x.shape[-1]).contiguous()
    out = (
        torch.empty((flat.shape[0], module.out_features), device=x.device, dtype=x.dtype)
        if allocate_output
        else None
    )
    return flat, out


def _validate_layout(module, scheme: str) -> None:
    n, k = module.out_features, module.in_features
    if scheme == "fp8":
        if tuple(module.weight.shape) != (n, k):
            raise ValueError(f"FP8 weight shape {tuple(module.weight.shape)} != {(n, k)}")
        if module.weight.dtype != torch.float8_e4m3fn:
            raise ValueError(f"FP8 weight dtype {module.weight.dtype} != float8_e4m3fn")
        if module.weight_scale.numel() not in (1, n):
            raise ValueError(
                "FP8 weight_scale must be scalar or per-output-channel, got "
                f"{tuple(module.weight_scale.shape)}"
            )
        if not module.activation_dynamic and module.input_scale.numel() != 1:
            raise ValueError("static FP8 input_scale must be scalar")
    elif scheme == "int8":
        if tuple(module.weight.shape) != (n, k):
            raise ValueError(f"INT8 weight shape {tuple(module.weight.shape)} != {(n, k)}")
        if module.weight.dtype != torch.int8:
            raise ValueError(f"INT8 weight dtype {module.weight.dtype} != int8")
        if module.weight_scale.numel() != n:
            raise ValueError("INT8 weight_scale must be per-output-channel")
    elif scheme == "awq":
        expected = ((k, n // 8), (k // module.group_size, n // 8), (k // module.group_size, n))
        actual = tuple(tuple(t.shape) for t in (module.qweight, module.qzeros, module.scales))
        if actual != expected:
            raise ValueError(f"AWQ packed layout {actual} != {expected}")
    elif scheme == "gptq":
        groups = -(-k // module.group_size)
        expected = ((k // 8, n), (groups, n // 8), (groups, n), (k,))
        actual = tuple(
            tuple(t.shape) for t in (module.qweight, module.qzeros, module.scales, module.g_idx)
        )
        if actual != expected:
            raise ValueError(f"GPTQ packed layout {actual} != {expected}")
    elif scheme == "fp8_block":
        expected = ((n, k), (-(-n // 128), -(-k // 128)))
        actual = (tuple(module.weight.shape), tuple(module.weight_scale_inv.shape))
        if actual != expected:
            raise ValueError(f"block FP8 layout {actual} != {expected}")
    if scheme in ("awq", "gptq") and module.scales.dtype != torch.float16:
        raise RuntimeError(
            f"{scheme} kernels consume fp16 checkpoint scales, got {module.scales.dtype}"
        )


def _f32(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    return t.contiguous()


def _bias(module, add_bias: bool) -> torch.Tensor | None:
    if not add_bias or module.bias is None:
        return None
    return module.bias.contiguous()


def _workspace(device: torch.device, nbytes: int = 0) -> torch.Tensor:
    return _native.workspace(device, nbytes)


@lru_cache(maxsize=4096)
def _workspace_bytes(entry: str, device_index: int, *shape: int) -> int:
    """A workspace-size entry point's answer for one shape (a pure function of
    the shape and of the device's CU count, fixed for the process)."""

    return int(getattr(_native.library(), entry)(*shape))


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _w8a8_linear_workspace(device: torch.device, m: int, n: int, k: int) -> torch.Tensor:
    """Workspace for a fused W8A8 call of this shape: the quantized rows and
    their scales (when they are staged) and every split-K form's partials."""

    need = _workspace_bytes("kq_w8a8_linear_workspace_size", _device_index(device), m, n, k)
    return _workspace(device, need)


def _w4_workspace(device: torch.device, m: int, n: int, k: int, mode: int) -> torch.Tensor:
    need = _workspace_bytes("kq_w4a16_workspace_size", _device_index(device), m, n, k, mode)
    return _workspace(device, need)


def _quantize_activation(
    flat: torch.Tensor,
    dtype: torch.dtype,
    quant_max: float,
    static_scale: torch.Tensor | None = None,
    row_scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token quantization of ``flat [M, K]`` -> (int8 or e4m3 ``[M, K]``, fp32 ``[M, 1]``)."""

    if static_scale is not None and row_scale is not None:
        raise ValueError("activation quantization accepts one scale source")
    if dtype not in (torch.int8, torch.float8_e4m3fn):
        raise RuntimeError(f"unsupported activation quantization dtype {dtype}")
    rows, k = flat.shape
    quantized = torch.empty((rows, k), device=flat.device, dtype=dtype)
    scales = torch.empty((rows, 1), device=flat.device, dtype=torch.float32)
    stream = _native.stream_handle(flat.device)
    if dtype is torch.int8:
        if static_scale is not None or row_scale is not None or quant_max != 127.0:
            raise ValueError("INT8 activation quantization is dynamic per token with max 127")
        _native.call(
            "kq_act_quant_i8",
            flat.data_ptr(), _native.dtype_code(flat.dtype), rows, k, flat.stride(0),
            quantized.data_ptr(), scales.data_ptr(), stream,
        )
        return quantized, scales
    if quant_max != 448.0:
        raise ValueError("FP8 e4m3 activation quantization uses max 448")
    mode, source = 0, None
    if row_scale is not None:
        mode, source = 2, _f32(row_scale.reshape(rows, 1).to(flat.device))
    elif static_scale is not None:
        mode, source = 1, _f32(static_scale.to(flat.device))
    _native.call(
        "kq_act_quant_fp8",
        flat.data_ptr(), _native.dtype_code(flat.dtype), rows, k, flat.stride(0),
        _native.ptr(source), mode, quantized.data_ptr(), scales.data_ptr(), stream,
    )
    return quantized, scales


def fp8_activation_amax(x: torch.Tensor) -> torch.Tensor:
    """Per-token fp32 amax ``[..., 1]`` without an fp32 activation temporary."""

    _native.library()
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"activation amax supports float16/bfloat16, got {x.dtype}")
    flat = x.reshape(-1, x.shape[-1]).contiguous()
    out = torch.empty((flat.shape[0], 1), device=flat.device, dtype=torch.float32)
    _native.call(
        "kq_row_amax",
        flat.data_ptr(), _native.dtype_code(flat.dtype), flat.shape[0], flat.shape[1],
        flat.stride(0), out.data_ptr(), _native.stream_handle(flat.device),
    )
    return out.reshape(*x.shape[:-1], 1)


def fp8_linear_forward(
    x: torch.Tensor,
    module,
    activation_scale: torch.Tensor | None = None,
    *,
    add_bias: bool = True,
) -> torch.Tensor:
    """FP8 W8A8: per-token (dynamic, static ``input_scale`` or given per-row
    ``activation_scale``) e4m3 quantization of ``x`` and the GEMM in one C call
    (small decode batches quantize inside the GEMM launch)."""

    flat, out = _prepare(x, module, "fp8")
    input_scale = None if module.activation_dynamic else module.input_scale
    if input_scale is not None and activation_scale is not None:
        raise ValueError("activation quantization accepts one scale source")
    m, k = flat.shape
    mode, source = 0, None
    if activation_scale is not None:
        mode, source = 2, _f32(activation_scale.reshape(m, 1).to(flat.device))
    elif input_scale is not None:
        mode, source = 1, _f32(input_scale.to(flat.device))
    weight_scale = _f32(module.weight_scale)
    bias = _bias(module, add_bias)
    ws = _w8a8_linear_workspace(x.device, m, module.out_features, k)
    _native.call(
        "kq_w8a8_fp8_linear",
        flat.data_ptr(), _native.dtype_code(flat.dtype), flat.stride(0), _native.ptr(source), mode,
        module.weight.data_ptr(), weight_scale.data_ptr(), int(weight_scale.numel() != 1),
        _native.ptr(bias), _native.dtype_code(None if bias is None else bias.dtype), out.data_ptr(),
        _native.dtype_code(x.dtype), m, module.out_features, k, ws.data_ptr(), ws.numel(),
        _native.stream_handle(x.device),
    )
    return out.reshape(*x.shape[:-1], module.out_features)


def int8_linear_forward(x: torch.Tensor, module, *, add_bias: bool = True,
                        accumulators: torch.Tensor | None = None) -> torch.Tensor:
    """INT8 W8A8: per-token int8 quantization of ``x`` and the GEMM in one C
    call.  ``accumulators`` (int32 ``[M, N]``, optional) receives the raw int32
    dot products for bit-exact checks."""

    flat, out = _prepare(x, module, "int8")
    weight_scale = _f32(module.weight_scale)
    bias = _bias(module, add_bias)
    m, k = flat.shape
    if accumulators is not None and (
        accumulators.dtype != torch.int32
        or tuple(accumulators.shape) != (m, module.out_features)
        or not accumulators.is_contiguous()
        or accumulators.device != x.device
    ):
        raise ValueError("accumulators must be a contiguous int32 [M, N] tensor on the device")
    ws = _w8a8_linear_workspace(x.device, m, module.out_features, k)
    _native.call(
        "kq_w8a8_i8_linear",
        flat.data_ptr(), _native.dtype_code(flat.dtype), flat.stride(0), module.weight.data_ptr(),
        weight_scale.data_ptr(), _native.ptr(bias),
        _native.dtype_code(None if bias is None else bias.dtype), out.data_ptr(),
        _native.dtype_code(x.dtype), _native.ptr(accumulators), m, module.out_features, k,
        ws.data_ptr(), ws.numel(), _native.stream_handle(x.device),
    )
    return out.reshape(*x.shape[:-1], module.out_features)


GIDX_UNIFORM = 0
GIDX_PERMUTED = 1
GIDX_PER_K = 2


class TiledOperand(NamedTuple):
    """A W4A16 weight as the tiled kernels read it: ``tiles`` (flat int32,
    ``kq_w4a16_tile_weights``) and the ``zeros`` / ``zero_offset`` arguments
    the tiled GEMM takes with it (``zeros`` None: one zero, ``zero_offset``,
    for every group and column)."""

    tiles: torch.Tensor
    zeros: torch.Tensor | None
    zero_offset: int


def _one_zero(qzeros: torch.Tensor) -> int | None:
    """The nibble every word of natural-order ``qzeros`` repeats, or None
    (one host read at load time)."""

    flat = qzeros.reshape(-1)
    nibble = int(flat[0].item()) & 0xF
    word = nibble * 0x11111111
    word = word - (1 << 32) if word >= (1 << 31) else word
    return nibble if bool((flat == word).all().item()) else None


def tile_operand(qweight: torch.Tensor, src_format: int, perm: torch.Tensor | None,
                 qzeros: torch.Tensor, zero_offset: int, scales: torch.Tensor, n: int, k: int,
                 group: int, device: torch.device) -> TiledOperand | None:
    """The tiled operand of ``kq_w4a16_tile_weights``: the [column
    tile][ceil(K/128) stages x 16 packed rows][16 columns] words in lane-major
    stage order, then the per-tile scale/zero table; ``qzeros`` is in natural
    nibble order.  When every zero is the same (symmetric checkpoints) the
    operand is built with one zero (``qzeros`` null in the C ABI): the decode
    GEMV then reads 2 bytes of scale per group and column and no zeros.  None
    for a shape the tiled kernels do not take (``kq_w4a16_tiled_words``)."""

    nibble = _one_zero(qzeros)
    one = nibble is not None
    words = int(_native.library().kq_w4a16_tiled_words(n, k, group, int(one)))
    if words < 0:
        return None
    tiles = torch.empty(words, dtype=torch.int32, device=device)
    zeros, zoff = (None, nibble + zero_offset) if one else (qzeros, zero_offset)
    _native.call(
        "kq_w4a16_tile_weights", qweight.data_ptr(), src_format, _native.ptr(perm),
        _native.ptr(zeros), zoff, scales.data_ptr(), tiles.data_ptr(), n, k, group,
        _native.stream_handle(device),
    )
    return TiledOperand(tiles, zeros, zoff)


def _refuse_under_capture(scheme: str) -> None:
    """Building derived W4A16 operands allocates and (GPTQ) compares g_idx on
    the host; neither may happen while a stream is capturing a graph."""

    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"{scheme} derived operands are missing or stale during graph capture; run the "
            "module once eagerly (after any weight update) before capturing"
        )


def awq_natural_zeros(qzeros: torch.Tensor, n: int, device: torch.device) -> torch.Tensor:
    """AWQ ``qzeros`` in natural nibble order (``kq_awq_natural_zeros``)."""

    natural = torch.empty_like(qzeros)
    _native.call("kq_awq_natural_zeros", qzeros.data_ptr(), natural.data_ptr(), n, qzeros.shape[0],
                 _native.stream_handle(device))
    return natural


def _awq_operands(module, device: torch.device) -> TiledOperand | None:
    """The tiled operand of an AWQ module, or None.

    The W4A16 kernels stream 16-column tiles of K-packed words
    (``kq_w4a16_tile_weights``); shapes with ``k % 8 == 0`` and
    ``group_size % 8 == 0`` get that derived, non-persistent copy (plus the
    zeros in natural nibble order), rebuilt when a source tensor's version
    changes.  Checkpoint buffers stay untouched, as for the reference's derived
    operands (quant_gemm_gpu.py:802-850).  Other shapes run on the checkpoint
    layout.
    """

    qweight, qzeros, scales = module.qweight, module.qzeros, module.scales
    k, n, group = module.in_features, module.out_features, module.group_size
    if k % 8 != 0 or group % 8 != 0:
        return None
    key = (id(qweight), qweight._version, id(qzeros), qzeros._version, id(scales),
           scales._version, str(device))
    cached = module.__dict__.get("_kq_awq_operands")
    if cached is not None and cached[0] == key:
        return cached[1]
    _refuse_under_capture("AWQ")
    result = tile_operand(qweight, 0, None, awq_natural_zeros(qzeros, n, device), 0, scales, n, k,
                          group, device)
    object.__setattr__(module, "_kq_awq_operands", (key, result))
    return result


def awq_linear_forward(x: torch.Tensor, module, *, add_bias: bool = True) -> torch.Tensor:
    flat, out = _prepare(x, module, "awq")
    bias = _bias(module, add_bias)
    m, k = flat.shape
    ws = _w4_workspace(x.device, m, module.out_features, k, GIDX_UNIFORM)
    tiled = _awq_operands(module, x.device)
    common = (
        _native.ptr(bias), _native.dtype_code(None if bias is None else bias.dtype),
        out.data_ptr(), m, module.out_features, k, module.group_size, ws.data_ptr(), ws.numel(),
        _native.stream_handle(x.device),
    )
    if tiled is not None:
        _native.call(
            "kq_w4a16_tiled_gemm",
            flat.data_ptr(), _native.dtype_code(flat.dtype), tiled.tiles.data_ptr(),
            _native.ptr(tiled.zeros), tiled.zero_offset, module.scales.data_ptr(), None, *common,
        )
    else:
        _native.call(
            "kq_w4a16_awq_gemm",
            flat.data_ptr(), _native.dtype_code(flat.dtype), module.qweight.data_ptr(),
            module.qzeros.data_ptr(), module.scales.data_ptr(), *common,
        )
    return out.reshape(*x.shape[:-1], module.out_features)


def _gptq_operands(module, device: torch.device):
    """(gidx_mode, weight operand, perm or None) for a GPTQ module: the
    operand is a ``TiledOperand`` for the uniform and act-order modes, else
    the checkpoint ``qweight``.

    ``g_idx == k // group_size`` and an act-order ``g_idx`` whose stable sort
    groups every ``group_size`` rows together run on a derived, non-persistent
    tiled copy of ``qweight`` (``kq_w4a16_tile_weights``; for act-order the
    rows are K-permuted by that sort and ``x`` is gathered through it), rebuilt
    when a source tensor's version changes.  Any other ``g_idx`` uses the
    per-element group path on the checkpoint buffers.
    """

    g_idx, qweight, qzeros, scales = module.g_idx, module.qweight, module.qzeros, module.scales
    key = (id(g_idx), g_idx._version, id(qweight), qweight._version, id(qzeros), qzeros._version,
           id(scales), scales._version, str(device))
    cached = module.__dict__.get("_kq_gptq_operands")
    if cached is not None and cached[0] == key:
        return cached[1]
    _refuse_under_capture("GPTQ")
    k, n, group = module.in_features, module.out_features, module.group_size
    mode, perm32 = gptq_group_mode(g_idx, k, group, device)
    result = (GIDX_PER_K, qweight, None)
    if mode != GIDX_PER_K:
        tiled = tile_operand(qweight, 1, perm32, qzeros, 1, scales, n, k, group, device)
        if tiled is not None:
            result = (mode, tiled, perm32)
    object.__setattr__(module, "_kq_gptq_operands", (key, result))
    return result


def gptq_group_mode(g_idx: torch.Tensor, k: int, group: int, device: torch.device):
    """(gidx_mode, perm int32 or None) of a GPTQ ``g_idx`` without building
    any operand: ``GIDX_UNIFORM`` when ``g_idx == k // group``,
    ``GIDX_PERMUTED`` with the stable argsort when that sort groups every
    ``group`` rows together (act-order), else ``GIDX_PER_K``."""

    if group % 8 != 0:
        return GIDX_PER_K, None
    natural = torch.arange(k, device=device, dtype=torch.int64) // group
    gi = g_idx.to(device=device, dtype=torch.int64)
    if torch.equal(gi, natural):
        return GIDX_UNIFORM, None
    perm = torch.argsort(gi, stable=True)
    if torch.equal(gi[perm], natural):
        return GIDX_PERMUTED, perm.to(torch.int32).contiguous()
    return GIDX_PER_K, None


def gptq_linear_forward(x: torch.Tensor, module, *, add_bias: bool = True) -> torch.Tensor:
    flat, out = _prepare(x, module, "gptq")
    mode, weight, perm = _gptq_operands(module, x.device)
    bias = _bias(module, add_bias)
    m, k = flat.shape
    ws = _w4_workspace(x.device, m, module.out_features, k, mode)
    common = (
        _native.ptr(bias), _native.dtype_code(None if bias is None else bias.dtype),
        out.data_ptr(), m, module.out_features, k, module.group_size, ws.data_ptr(), ws.numel(),
        _native.stream_handle(x.device),
    )
    if mode in (GIDX_UNIFORM, GIDX_PERMUTED):
        _native.call(
            "kq_w4a16_tiled_gemm",
            flat.data_ptr(), _native.dtype_code(flat.dtype), weight.tiles.data_ptr(),
            _native.ptr(weight.zeros), weight.zero_offset, module.scales.data_ptr(),
            _native.ptr(perm), *common,
        )
    else:
        g_idx = module.g_idx if module.g_idx.dtype == torch.int32 else module.g_idx.to(torch.int32)
        _native.call(
            "kq_w4a16_gptq_gemm",
            flat.data_ptr(), _native.dtype_code(flat.dtype), weight.data_ptr(),
            module.qzeros.data_ptr(), module.scales.data_ptr(), g_idx.data_ptr(), None, mode,
            *common,
        )
    return out.reshape(*x.shape[:-1], module.out_features)


def quantize_activation_blocks(flat: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per token per 128-wide K block e4m3 quantization of ``flat [M, K]``:
    (e4m3 ``[M, K]``, fp32 ``[M, ceil(K/128)]``), ``s = max(amax, 1e-12)/448``."""

    rows, k = flat.shape
    quantized = torch.empty((rows, k), device=flat.device, dtype=torch.float8_e4m3fn)
    scales = torch.empty((rows, -(-k // 128)), device=flat.device, dtype=torch.float32)
    _native.call(
        "kq_act_quant_fp8_blocks", flat.data_ptr(), _native.dtype_code(flat.dtype), rows, k,
        flat.stride(0), quantized.data_ptr(), scales.data_ptr(), _native.stream_handle(flat.device),
    )
    return quantized, scales


def block_fp8_linear_forward(x: torch.Tensor, module, *, add_bias: bool = True) -> torch.Tensor:
    """128x128 block-scaled FP8 linear: dynamic 1x128 activation blocks, e4m3
    MFMA per block scaled by ``s_x * s_w`` in fp32, output in ``x.dtype``."""

    flat, out = _prepare(x, module, "fp8_block")
    m, k = flat.shape
    if k % 128 != 0:
        raise ValueError(f"block FP8 kernel needs in_features % 128 == 0, got {k}")
    bias = _bias(module, add_bias)
    x_q, x_scale = quantize_activation_blocks(flat)
    scale_inv = _f32(module.weight_scale_inv)
    _native.call(
        "kq_block_fp8_gemm", x_q.data_ptr(), x_scale.data_ptr(), module.weight.data_ptr(),
        scale_inv.data_ptr(), _native.ptr(bias),
        _native.dtype_code(None if bias is None else bias.dtype), out.data_ptr(),
        _native.dtype_code(out.dtype), m, module.out_features, k, _native.stream_handle(x.device),
    )
    return out.reshape(*x.shape[:-1], module.out_features)


_DISPATCH = {
    "fp8": fp8_linear_forward,
    "int8": int8_linear_forward,
    "awq": awq_linear_forward,
    "gptq": gptq_linear_forward,
    "fp8_block": block_fp8_linear_forward,
}


def linear_forward(x: torch.Tensor, module, *, add_bias: bool = True) -> torch.Tensor:
    scheme = getattr(module, "quant_scheme", None)
    if scheme not in _DISPATCH:
        raise RuntimeError(f"no fused GPU kernel registered for {scheme!r}")
    return _DISPATCH[scheme](x, module, add_bias=add_bias)
