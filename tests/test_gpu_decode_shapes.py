"""Decode-sized W4A16 calls (M <= 16) at the projection shapes of the models
the reference serves (Llama-3-8B: down_proj N=4096 K=14336, k_proj N=1024
K=4096; Qwen2-7B: q_proj N=K=3584, down_proj N=3584 K=18944, k_proj N=512
K=3584; kairyu/models/layers.py:212-241, attention.py:51-94) against the CPU
oracle, every output column.

These reach the decode GEMV's generalized forms: K = 3584 (a 16-wave window
grid with inactive waves past K), fewer 16-column units than CUs (one unit
per workgroup), K split across workgroups (K = 14336, 18944: chunks of 4096;
K % 256 == 128: one-stage windows and chunks of 2048) with the split-K
reduce, and a unit half past N.
Formats: AWQ (asymmetric zeros), GPTQ act-order with the symmetric zero (the
one-zero operand), GPTQ with per-column zeros; fp16 and bf16 activations.
Per-element bound of ``gpu_helpers.check_w4a16``.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import banner, check_w4a16
from kairyu_amd import workloads

pytestmark = pytest.mark.gpu

SHAPES = [
    ("llama down", 4096, 14336),
    ("llama k_proj", 1024, 4096),
    ("qwen q_proj", 3584, 3584),
    ("qwen down", 3584, 18944),
    ("qwen k_proj", 512, 3584),
    # 33 stages (K % 256 == 128): one-stage windows, three K chunks of 44 steps
    ("odd stages", 2048, 4224),
    # 17 stages: one-stage windows, two K chunks (36 and 32 steps)
    ("two chunks", 1024, 2176),
    # N % 16 == 8: the last unit half past N
    ("ragged N", 520, 4096),
]


def _module(fmt: str, m: int, n: int, k: int, cuda, x_dtype):
    if fmt == "awq":
        return workloads.awq_layer(m=m, n=n, k=k, device=cuda, x_dtype=x_dtype)
    wl = workloads.gptq_layer(m=m, n=n, k=k, device=cuda, x_dtype=x_dtype, act_order=fmt == "gptq-ao")
    if fmt == "gptq-zeros":
        from kairyu_amd.quant import gptq as gptq_format

        g = torch.Generator().manual_seed(n + k)
        zeros = torch.randint(0, 16, tuple(wl.module.scales.shape), generator=g)
        wl.module.qzeros.copy_(gptq_format.pack_gptq_cols(zeros).to(cuda))
    return wl


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0].replace(" ", "-") for s in SHAPES])
@pytest.mark.parametrize("fmt,m,x_dtype", [
    ("awq", 16, torch.float16),
    ("gptq-ao", 1, torch.float16),
    ("gptq-ao", 16, torch.float16),
    ("gptq-zeros", 5, torch.bfloat16),
])
def test_decode_projection_shapes_match_oracle(cuda, shape, fmt, m, x_dtype):
    label, n, k = shape
    banner(f"decode {label} N={n} K={k} {fmt} M={m} {x_dtype}")
    wl = _module(fmt, m, n, k, cuda, x_dtype)
    out = wl.module(wl.x)
    assert out.dtype == x_dtype and out.shape == (m, n)
    check_w4a16(out, wl.module, wl.x.cpu(), label=f"{label} {fmt} M={m}")
    # a second call on the cached operands gives the same bits
    assert torch.equal(wl.module(wl.x), out)


W8_SHAPES = [s for s in SHAPES if s[0] in ("llama down", "llama k_proj", "qwen q_proj", "qwen down", "qwen k_proj")]


@pytest.mark.parametrize("shape", W8_SHAPES, ids=[s[0].replace(" ", "-") for s in W8_SHAPES])
@pytest.mark.parametrize("fmt,m", [("fp8", 1), ("fp8", 16), ("int8", 1), ("int8", 16)])
def test_w8a8_decode_projection_shapes_match_oracle(cuda, shape, fmt, m):
    """W8A8 decode at the same shapes: tile counts from one per CU (N = 3584,
    4096) down to 32 (N = 512), where the decode kernel takes 8 or 16 waves,
    and the one-row call that quantizes inside the decode launch.  FP8 within
    the per-element bound; INT8 accumulators and bf16 output bit-exact."""
    import numpy as np

    from gpu_helpers import bits, check_fp8, np32
    from kairyu_amd.kernels import quant_gemm_hip as hip
    from oracle import linear as olinear
    from oracle.numerics import bf16_bits

    label, n, k = shape
    banner(f"decode {label} N={n} K={k} {fmt} M={m}")
    if fmt == "fp8":
        wl = workloads.fp8_layer(m=m, n=n, k=k, device=cuda)
        out = wl.module(wl.x)
        check_fp8(out, wl.x.cpu(), wl.module, label=f"{label} fp8 M={m}")
        return
    wl = workloads.int8_layer(m=m, n=n, k=k, device=cuda)
    module = wl.module
    out = module(wl.x)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    out_acc = hip.int8_linear_forward(wl.x, module, accumulators=acc)
    assert torch.equal(out.view(torch.int16), out_acc.view(torch.int16))
    expected, _, _, eacc = olinear.int8_forward(np32(wl.x), module.weight.cpu().numpy(),
                                                np32(module.weight_scale), None)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), eacc)
    assert np.array_equal(bits(out), bf16_bits(expected).view(np.int16))


@pytest.mark.parametrize("n,k", [(4096, 14336), (3584, 18944), (2048, 4224)])
def test_long_k_act_order_decode_fits_the_exact_workspace(cuda, n, k):
    """Act-order decode with K split across workgroups needs the gathered x
    and the fp32 split partials in one workspace: the call runs in exactly
    kq_w4a16_workspace_size bytes (an upper bound over the shape's paths; a
    guard region behind it stays untouched), gives the module forward's bits,
    and a buffer smaller than the gathered x alone is refused."""
    from kairyu_amd import _native
    from kairyu_amd.kernels import quant_gemm_hip as hip

    m = 16
    banner(f"exact workspace act-order decode N={n} K={k}")
    wl = workloads.gptq_layer(m=m, n=n, k=k, device=cuda, act_order=True)
    module = wl.module
    expected = module(wl.x)
    mode, weight, perm = hip._gptq_operands(module, cuda)
    need = int(_native.library().kq_w4a16_workspace_size(m, n, k, mode))
    guard = 1 << 16
    buf = torch.full((need + guard,), 0x5A, dtype=torch.uint8, device=cuda)
    out = torch.empty_like(expected)

    def call(nbytes):
        _native.call("kq_w4a16_tiled_gemm", wl.x.data_ptr(), _native.dtype_code(wl.x.dtype),
                     weight.tiles.data_ptr(), _native.ptr(weight.zeros), weight.zero_offset,
                     module.scales.data_ptr(), _native.ptr(perm), None, _native.DTYPE_NONE, out.data_ptr(),
                     m, n, k, module.group_size, buf.data_ptr(), nbytes, _native.stream_handle(cuda))

    call(need)
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16))
    assert bool((buf[need:] == 0x5A).all())
    with pytest.raises(RuntimeError, match="workspace"):
        call(m * k)  # half the fp16 gathered x
