"""ctypes binding of ``libkairyu_quant.so`` (C ABI in ``include/kairyu_quant.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded: both then share
one device context and torch's streams can be passed straight through.  There
is no fallback of any kind: a missing or unloadable library raises
``RuntimeError`` at the first device call.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libkairyu_quant.so"

KQ_OK = 0
KQ_EINVAL = 1
KQ_EUNSUPPORTED = 2
KQ_ELAUNCH = 3
KQ_EWORKSPACE = 4

DTYPE_NONE = -1
DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

# split-K partial sums and the act-order activation gather; 32 MiB covers
# every decode shape at its preferred split count.
DEFAULT_WORKSPACE_BYTES = 32 * 1024 * 1024

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

_SIGNATURES: dict[str, list] = {
    "kq_version": [],
    "kq_last_error": [],
    "kq_device_supported": [_I],
    "kq_row_amax": [_P, _I, _I64, _I64, _I64, _P, _P],
    "kq_act_quant_i8": [_P, _I, _I64, _I64, _I64, _P, _P, _P],
    "kq_act_quant_fp8": [_P, _I, _I64, _I64, _I64, _P, _I, _P, _P, _P],
    "kq_w8a8_i8_gemm": [_P, _P, _P, _P, _P, _I, _P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "kq_w8a8_fp8_gemm": [_P, _P, _P, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _P, _SZ, _P],
    "kq_w8a8_workspace_size": [_I64, _I64, _I64],
    "kq_w8a8_i8_linear": [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "kq_w8a8_fp8_linear": [
        _P, _I, _I64, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _P, _SZ, _P,
    ],
    "kq_w8a8_linear_workspace_size": [_I64, _I64, _I64],
    "kq_w8a8_i8_swiglu_linear": [_P, _I, _I64, _P, _P, _P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "kq_w8a8_fp8_swiglu_linear": [
        _P, _I, _I64, _P, _I, _P, _P, _I, _P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P,
    ],
    "kq_w8a8_swiglu_workspace_size": [_I64, _I64, _I64],
    "kq_w4a16_awq_gemm": [_P, _I, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _P, _SZ, _P],
    "kq_w4a16_gptq_gemm": [
        _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _P, _I64, _I64, _I64, _I, _P, _SZ, _P,
    ],
    "kq_gptq_permute_qweight": [_P, _P, _P, _I64, _I64, _P],
    "kq_w4a16_tile_weights": [_P, _I, _P, _P, _I, _P, _P, _I64, _I64, _I, _P],
    "kq_w4a16_tiled_words": [_I64, _I64, _I, _I],
    "kq_awq_natural_zeros": [_P, _P, _I64, _I64, _P],
    "kq_w4a16_tiled_gemm": [
        _P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _P, _SZ, _P,
    ],
    "kq_w4a16_tiled_gemm_noalloc": [
        _P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _P,
    ],
    "kq_w4a16_workspace_size": [_I64, _I64, _I64, _I],
    "kq_w4a16_tiled_swiglu_gemm": [
        _P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _P, _SZ, _P,
    ],
    "kq_w4a16_swiglu_workspace_size": [_I64, _I64, _I64, _I],
    "kq_swiglu": [_P, _I64, _I, _I, _P, _I64, _I64, _P],
    "kq_moe_route_topk": [_P, _I, _I64, _I64, _I, _I, _P, _P, _P],
    "kq_act_quant_fp8_blocks": [_P, _I, _I64, _I64, _I64, _P, _P, _P],
    "kq_block_fp8_gemm": [_P, _P, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P],
    "kq_moe_workspace_size": [_I64, _I64, _I64, _I64, _I],
    "kq_peak_stream_read": [_P, _I64, _I, _P, _P],
    "kq_peak_mfma": [_I, _I64, _I, _P, _P],
    "kq_moe_block_fp8_experts": [
        _P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P,
    ],
    "kq_moe_routed_block_fp8_experts": [
        _P, _I, _I, _P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P,
    ],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        path = Path(os.environ.get("KAIRYU_AMD_LIB", LIB_PATH))
        if not path.is_file():
            _load_error = f"{path} is not built; run kairyu_amd.build.build() (hipcc, gfx950)"
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as error:
            _load_error = f"cannot load {path}: {error}"
            raise RuntimeError(_load_error) from error
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = {"kq_last_error": ctypes.c_char_p,
                          "kq_w4a16_workspace_size": ctypes.c_size_t,
                          "kq_w4a16_swiglu_workspace_size": ctypes.c_size_t,
                          "kq_w4a16_tiled_words": ctypes.c_int64,
                          "kq_w8a8_workspace_size": ctypes.c_size_t,
                          "kq_w8a8_linear_workspace_size": ctypes.c_size_t,
                          "kq_w8a8_swiglu_workspace_size": ctypes.c_size_t,
                          "kq_moe_workspace_size": ctypes.c_size_t}.get(name, ctypes.c_int)
        _lib = lib
        return lib


def library() -> ctypes.CDLL:
    """The loaded kernel library; raises RuntimeError when it is unavailable."""

    return _load()


def exported_symbols() -> tuple[str, ...]:
    return tuple(_SIGNATURES)


def call(name: str, *args) -> None:
    """Invoke one C entry point and map its status to the reference's exceptions."""

    lib = _load()
    status = getattr(lib, name)(*args)
    if status == KQ_OK:
        return
    message = lib.kq_last_error().decode(errors="replace")
    if status == KQ_EINVAL:
        raise ValueError(f"{name}: {message}")
    raise RuntimeError(f"{name} failed ({status}): {message}")


def dtype_code(dtype: torch.dtype | None) -> int:
    if dtype is None:
        return DTYPE_NONE
    if dtype is torch.float16:
        return DTYPE_F16
    if dtype is torch.bfloat16:
        return DTYPE_BF16
    if dtype is torch.float32:
        return DTYPE_F32
    raise RuntimeError(f"unsupported dtype {dtype} at the kernel boundary")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """torch's current stream on `device` (the capture stream inside graph
    capture) as a raw hipStream_t, read without building a Stream object."""

    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


_supported: dict[int, bool] = {}


def device_supported(index: int) -> bool:
    if index not in _supported:
        _supported[index] = bool(_load().kq_device_supported(index))
    return _supported[index]


class WorkspacePool:
    """Per-device scratch buffers (split-K partials, act-order activation
    gather, MoE intermediates), one per device, reused by every call.

    Growth is geometric: a call needing more than the current buffer gets
    ``max(need, 2 * current)`` bytes, so a sequence of ever larger calls
    allocates O(log(need)) times.  A buffer handed out while the stream was
    capturing a graph may be referenced by that graph, so once outgrown it is
    retained until the process ends; the retained buffers of one device sum to
    less than its current buffer (each is at most half the next).  Any other
    outgrown buffer is released after a device synchronization (kernels still
    queued on it must finish before torch's allocator can hand it out again).
    Calls sharing the buffer must be ordered on one stream, like the engine's
    single-stream decode loop; grow it with an eager call of the largest shape
    before capturing.
    """

    def __init__(self, allocate, capturing, synchronize, minimum: int = DEFAULT_WORKSPACE_BYTES):
        self._allocate = allocate
        self._capturing = capturing
        self._synchronize = synchronize
        self._minimum = minimum
        self._buffers: dict[int, torch.Tensor] = {}
        self._captured: dict[int, bool] = {}
        self.retained: list[torch.Tensor] = []

    @staticmethod
    def grown_size(current: int, need: int, minimum: int) -> int:
        return max(need, 2 * current, minimum)

    def get(self, index: int, nbytes: int) -> torch.Tensor:
        buffer = self._buffers.get(index)
        capturing = bool(self._capturing(index))
        if buffer is None or buffer.numel() < nbytes:
            current = 0 if buffer is None else buffer.numel()
            if buffer is not None:
                if self._captured.get(index, False) or capturing:
                    self.retained.append(buffer)
                else:
                    self._synchronize(index)
            buffer = self._allocate(index, self.grown_size(current, nbytes, self._minimum))
            self._buffers[index] = buffer
            self._captured[index] = False
        if capturing:
            self._captured[index] = True
        return buffer


def _allocate_device(index: int, nbytes: int) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", index))


def _capturing(index: int) -> bool:
    return torch.cuda.is_current_stream_capturing()


def _synchronize(index: int) -> None:
    torch.cuda.synchronize(index)


_pool = WorkspacePool(_allocate_device, _capturing, _synchronize)


def workspace(device: torch.device, nbytes: int = DEFAULT_WORKSPACE_BYTES) -> torch.Tensor:
    """The device's scratch buffer, at least ``nbytes`` long (``WorkspacePool``)."""

    index = device.index if device.index is not None else torch.cuda.current_device()
    return _pool.get(index, nbytes)
