"""``kq_w4a16_tiled_gemm_noalloc`` (the allocation-free form of
``kq_w4a16_tiled_gemm``, scratch in a fixed per-device array) called through
the C ABI: bit-identical to the workspace entry point on the same operands,
call after call with shrinking inputs (the array keeps the previous call's
contents), within the oracle's per-element bound, and shapes whose scratch
exceeds the fixed size are rejected before anything is launched."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import banner, check_w4a16
from kairyu_amd import _native
from kairyu_amd.kernels import quant_gemm_hip as hip
from test_gpu_w4a16 import _awq_module, _gptq_module

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _operands(module, cuda):
    if hasattr(module, "g_idx"):
        mode, op, perm = hip._gptq_operands(module, cuda)
        assert mode in (hip.GIDX_UNIFORM, hip.GIDX_PERMUTED)
        return op.tiles, op.zeros, op.zero_offset, perm
    op = hip._awq_operands(module, cuda)
    return op.tiles, op.zeros, op.zero_offset, None


def _run(entry, module, x, cuda):
    tiles, zeros, zero_offset, perm = _operands(module, cuda)
    m, k = x.shape
    n = module.out_features
    out = torch.empty(m, n, device=cuda, dtype=x.dtype)
    bias = module.bias
    args = [x.data_ptr(), _native.dtype_code(x.dtype), tiles.data_ptr(), _native.ptr(zeros), zero_offset,
            module.scales.data_ptr(), _native.ptr(perm), _native.ptr(bias),
            _native.dtype_code(None if bias is None else bias.dtype), out.data_ptr(), m, n, k,
            module.group_size]
    if entry == "kq_w4a16_tiled_gemm":
        need = int(_native.library().kq_w4a16_workspace_size(m, n, k, 1 if perm is not None else 0))
        ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=cuda)
        args += [ws.data_ptr(), ws.numel()]
    _native.call(entry, *args, _native.stream_handle(cuda))
    return out


@pytest.mark.parametrize("fmt", ["gptq_act_order", "gptq", "awq"])
def test_noalloc_matches_workspace_entry_call_after_call(cuda, fmt):
    k, n, group = 4096, 2048, 128
    g = torch.Generator().manual_seed(41)
    if fmt == "awq":
        module = _awq_module(k, n, group=group, seed=41, random_packed=True)
    else:
        g_idx = ((torch.randperm(k, generator=g) if fmt == "gptq_act_order" else torch.arange(k)) // group)
        module = _gptq_module(k, n, group=group, seed=41, g_idx=g_idx.to(torch.int32), random_packed=True)
    module = module.to(cuda)
    # prefill (staged activations), then decode GEMV and skinny shapes, each
    # call smaller than the one before it
    for m, dtype in ((300, torch.float16), (64, torch.bfloat16), (16, torch.float16), (3, torch.bfloat16),
                     (1, torch.float16)):
        banner(f"noalloc {fmt} m={m} {dtype}")
        x = torch.randn(m, k, generator=g).to(dtype).to(cuda)
        got = _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda)
        want = _run("kq_w4a16_tiled_gemm", module, x, cuda)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (fmt, m)
        check_w4a16(got, module, x.cpu(), label=f"noalloc {fmt} m={m}")


def test_noalloc_rejects_shapes_beyond_the_fixed_scratch(cuda):
    module = _gptq_module(4096, 256, group=128, seed=42, random_packed=True,
                          g_idx=(torch.randperm(4096) // 128).to(torch.int32)).to(cuda)
    m = SCRATCH_BYTES // (4096 * 2) + 64          # act-order gather alone exceeds it
    assert int(_native.library().kq_w4a16_workspace_size(m, 256, 4096, 1)) > SCRATCH_BYTES
    x = torch.zeros(m, 4096, device=cuda, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="fixed"):
        _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda)
    # the array keeps working for a fitting call afterwards
    x = torch.randn(8, 4096, device=cuda, dtype=torch.float16)
    got = _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda)
    assert torch.equal(got, _run("kq_w4a16_tiled_gemm", module, x, cuda))


@pytest.mark.parametrize("m", [16, 64])
def test_noalloc_captured_in_a_graph_replays_the_eager_result(cuda, m):
    """One eager call (it resolves the array's device address), then the
    allocation-free call captured in a HIP graph: every replay, with other
    calls of the entry between replays overwriting the shared array, is
    bit-equal to the eager output (act-order gather and decode GEMV at
    m = 16, staged prefill at m = 64)."""
    k, n, group = 4096, 2048, 128
    g = torch.Generator().manual_seed(43)
    g_idx = (torch.randperm(k, generator=g) // group).to(torch.int32)
    module = _gptq_module(k, n, group=group, seed=43, g_idx=g_idx, random_packed=True).to(cuda)
    x = torch.randn(m, k, generator=g).to(torch.float16).to(cuda)
    other = torch.randn(m + 7, k, generator=g).to(torch.float16).to(cuda)
    banner(f"noalloc graph m={m}")
    eager = _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _run("kq_w4a16_tiled_gemm_noalloc", module, x, cuda)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), i
        _run("kq_w4a16_tiled_gemm_noalloc", module, other, cuda)  # eager work on the same array
        torch.cuda.synchronize()
