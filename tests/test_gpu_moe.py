"""Block-FP8 MoE and the dense block-FP8 linear on gfx950 against the CPU oracle.

Routing: expert indices exact (stable, ties to the smaller id), weights within
2e-6 relative (fp32 softmax; exp may differ from numpy's by an ulp).
Activation quantization (1x128 blocks): bytes and scales bit-exact.
Dense block-FP8 linear: every output within one ulp (plus an fp32
accumulation slack) of the fp64-accumulated oracle.  Routed experts
(``oracle.parity.moe_check``): every output within the reference's grouped-MoE
tolerance (atol 2e-2 + rtol 1e-2), the normwise maximum within 1e-2 at C5's
widths (2e-2 for the narrower synthetic layers, where one e4m3
re-quantization flip of the SwiGLU product moves an output by up to 1.4e-2 of
the largest output on the emulated device), every token row's and output
column's relative RMSE bounded, at least 95% of the outputs within eight ulps
(fp16 at C5's widths: 64, the same relative width) and relative RMSE <= 5e-3
(``tests/test_parity_bounds.py`` pins the criterion with planted mistakes).
Parity of the block-FP8 expert arithmetic is unpinned at the reference boundary (its hub kernel is not
vendored); every piece is pinned by the oracle's own tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import assert_moe_close, banner, check_block_fp8, np32
from kairyu_amd import _native
from kairyu_amd import moe as hmoe
from kairyu_amd import workloads
from kairyu_amd.kernels import quant_gemm_hip as hip
from kairyu_amd.quant.block_fp8 import quantize_block_fp8
from kairyu_amd.quant.linear import BlockFp8Linear
from oracle import formats, moe

pytestmark = pytest.mark.gpu


_DT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}
# normwise bound of the layers whose reductions are narrower than C5's (module docstring)
_NARROW = {"normwise": 2e-2}


def _covering_sample(idx: np.ndarray, experts: int, size: int, seed: int) -> np.ndarray:
    """Tokens that reach every routed expert's first row and the last row
    block (16 rows) of each of its row tiles, topped up with seeded others to
    ``size``.  Rows of an expert are its tokens in ascending order, tiles are
    320 rows when the routing averages more than 192 rows per expert, else
    256 (kq_moe.hip)."""
    tokens, top_k = idx.shape
    bm = 320 if tokens * top_k > 192 * experts else 256
    chosen = set()
    for e in range(experts):
        rows = np.nonzero((idx == e).any(axis=1))[0]
        if rows.size == 0:
            continue
        chosen.add(int(rows[0]))
        for start in range(0, rows.size, bm):
            chosen.add(int(rows[min(rows.size, start + bm) - 1]))
    rest = np.setdiff1d(np.arange(tokens), np.fromiter(chosen, np.int64))
    fill = max(0, size - len(chosen))
    extra = np.random.default_rng(seed).choice(rest, size=min(fill, rest.size), replace=False)
    return np.sort(np.concatenate([np.fromiter(chosen, np.int64), extra]))


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("experts,top_k", [(4, 1), (60, 2), (128, 8), (200, 8), (256, 8), (512, 8)])
@pytest.mark.parametrize("norm", [True, False])
def test_route_matches_oracle(cuda, dtype, experts, top_k, norm):
    g = torch.Generator().manual_seed(experts * 7 + top_k)
    logits = torch.randn(333, experts, generator=g)
    logits[::3] = torch.round(logits[::3] * 2) / 2  # many exact ties
    logits = logits.to(dtype)
    idx, w = hmoe.route_logits(logits.to(cuda), top_k, norm)
    oidx, ow = moe.route_topk(logits.float().numpy(), top_k, norm)
    assert np.array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("shape", [(37, 640), (5, 1000), (1, 128), (3, 4104)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_block_activation_quant_is_bit_exact(cuda, shape, dtype):
    g = torch.Generator().manual_seed(shape[1])
    x = (torch.randn(shape, generator=g) * 3).to(dtype)
    x[0, :7] = 0.0
    if shape[1] >= 256:
        x[-1, 128:256] = 0.0  # an all-zero block: scale 1e-12 / 448
    q, s = hip.quantize_activation_blocks(x.to(cuda))
    oq, os_ = formats.block_fp8_quantize_rows(x.float().numpy())
    assert np.array_equal(_bits(q), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


def test_block_activation_quant_edge_values_bit_exact(cuda):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 1024, generator=g) * 5
    x[0, :128:3] = -0.0                                  # signed zeros
    x[0, 128:256] = torch.randn(128, generator=g) * 1e-30
    x[0, 200] = 2.0                                      # the rest quantizes to +-0
    x[1, :128] = torch.tensor([1.0625, -1.1875, 0.017578125, 240.0]).repeat(32)
    x[1, 127] = 448.0                                    # s = 1: exact e4m3 ties
    x[2, 300] = float("inf")                             # block 2 of row 2: IEEE path
    x[3, 700] = float("nan")                             # block 5 of row 3: NaN scale
    x[3, 900:1024] = torch.randn(124, generator=g) * 1e37
    x = x.to(torch.bfloat16)
    q, s = hip.quantize_activation_blocks(x.to(cuda))
    with np.errstate(invalid="ignore", divide="ignore"):
        oq, os_ = formats.block_fp8_quantize_rows(x.float().numpy())
    assert np.array_equal(_bits(q), oq)
    # scales: bit-exact where finite; any NaN where the block holds a NaN
    np.testing.assert_array_equal(s.cpu().numpy(), os_)


@pytest.mark.parametrize("m", [1, 17, 130])
@pytest.mark.parametrize("n", [384, 200])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_block_fp8_linear_matches_oracle(cuda, m, n, dtype):
    k = 512
    g = torch.Generator().manual_seed(m * n)
    module = BlockFp8Linear(k, n, bias=True)
    q, s = quantize_block_fp8(torch.randn(n, k, generator=g) * 0.05)
    module.weight.copy_(q)
    module.weight_scale_inv.copy_(s)
    module.bias.data.normal_(generator=g)
    x = torch.randn(m, k, generator=g).to(dtype)
    out = module.to(cuda)(x.to(cuda))
    assert out.dtype == dtype
    check_block_fp8(out, x, module, label=f"dense m={m} n={n}")


def _pack(experts, hidden, inter, seed, device, std=0.05):
    g = torch.Generator().manual_seed(seed)
    q13, s13 = quantize_block_fp8(torch.randn(experts, 2 * inter, hidden, generator=g) * std)
    q2, s2 = quantize_block_fp8(torch.randn(experts, hidden, inter, generator=g) * std)
    return hmoe.GroupedBlockFp8Experts.from_tensors(q13.to(device), s13.to(device), q2.to(device), s2.to(device))


def _oracle_moe(pack, x, idx, w, tokens=None):
    sel = slice(None) if tokens is None else tokens
    dtype = "bfloat16" if x.dtype == torch.bfloat16 else "float16"
    return moe.moe_forward(x.float().numpy()[sel], idx[sel], w[sel], _bits(pack.w13), pack.s13.cpu().numpy(),
                           _bits(pack.w2), pack.s2.cpu().numpy(), dtype)


@pytest.mark.parametrize("cfg", [
    # tokens, hidden, inter, experts, top_k, dtype, experts used
    (40, 256, 256, 8, 2, torch.bfloat16, 8),
    (100, 384, 128, 16, 4, torch.float16, 7),     # most experts empty
    (7, 128, 384, 4, 4, torch.bfloat16, 4),       # top_k == experts
    (300, 512, 256, 32, 8, torch.bfloat16, 32),
    # experts with more rows than one row tile: 1000 rows each (320-row tiles:
    # 320, 320, 320 and 40) and ≈470 rows each (the routing averages 175 rows
    # over the 8 experts: 256-row tiles of 256 and ≈210)
    (1000, 256, 128, 4, 4, torch.bfloat16, 4),
    (700, 256, 256, 8, 2, torch.float16, 3),
])
def test_routed_block_fp8_experts_match_oracle(cuda, cfg):
    tokens, hidden, inter, experts, top_k, dtype, used = cfg
    banner(f"moe {cfg}")
    pack = _pack(experts, hidden, inter, seed=tokens + hidden, device=cuda)
    g = torch.Generator().manual_seed(tokens)
    x = torch.randn(tokens, hidden, generator=g).to(dtype)
    logits = torch.randn(tokens, experts, generator=g)
    logits[:, used:] = -1e4  # route only to the first `used` experts
    idx, w = hmoe.route_logits(logits.to(cuda), top_k)
    out = pack.forward(x.to(cuda), idx, w)
    assert out.dtype == dtype
    expected = _oracle_moe(pack, x, idx.cpu().numpy(), w.cpu().numpy())
    assert_moe_close(np32(out), expected, _DT[dtype], label=str(cfg), **_NARROW)


@pytest.mark.parametrize("tokens,top_k,experts", [
    (600, 8, 512),     # 19 sort chunks over 2 slices: runs of <= 16 chunks
    (1000, 8, 1024),   # 32 chunks, one slice: runs of <= 64 chunks
    (3000, 8, 1024),   # 94 chunks, one slice: the any-length scan
])
def test_sort_scan_forms_match_oracle(cuda, tokens, top_k, experts):
    """Every form of the expert-offset scan (by chunks per thread), with
    many experts and given top-k indices (each token's experts distinct).

    A token's result does not depend on the other tokens of the call (fixed
    K order per output, per-token quantization, slot-order combine), so the
    whole call must equal, bit for bit, the same tokens run 256 at a time
    (8 sort chunks: the short-run form); a token sample is checked against
    the oracle."""
    banner(f"moe sort tokens={tokens} top_k={top_k} experts={experts}")
    pack = _pack(experts, 128, 128, seed=tokens, device=cuda)
    g = torch.Generator().manual_seed(tokens + 1)
    x = torch.randn(tokens, 128, generator=g).to(torch.bfloat16)
    idx = torch.argsort(torch.rand(tokens, experts, generator=g), dim=1)[:, :top_k].to(torch.int32)
    w = torch.softmax(torch.randn(tokens, top_k, generator=g), dim=1)
    xd, idxd, wd = x.to(cuda), idx.to(cuda), w.to(cuda)
    out = pack.forward(xd, idxd, wd)
    parts = torch.cat([pack.forward(xd[i:i + 256], idxd[i:i + 256], wd[i:i + 256])
                       for i in range(0, tokens, 256)])
    assert torch.equal(out, parts)
    sample = np.random.default_rng(tokens).choice(tokens, size=64, replace=False)
    expected = _oracle_moe(pack, x, idx.numpy(), w.numpy(), tokens=sample)
    assert_moe_close(np32(out)[sample], expected, "bfloat16", label=f"sort {tokens}x{top_k} E={experts}",
                     **_NARROW)


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,ldtype,norm", [
    (333, 256, 128, 60, 6, torch.float32, True),     # 42 tokens (252 rows) per sort chunk
    (100, 128, 256, 4, 1, torch.bfloat16, False),    # top-1: 256 tokens per chunk, full softmax
    (257, 256, 128, 200, 8, torch.float16, True),    # 4 logits per lane, a one-token last chunk
    (64, 128, 128, 512, 8, torch.float32, False),    # 8 logits per lane; E > 256: the two-launch scan
    (9000, 128, 128, 128, 8, torch.float32, True),   # 282 chunks x 128 experts: past the one-launch scan
    (1, 128, 128, 8, 2, torch.bfloat16, True),
    (150, 128, 128, 64, 16, torch.bfloat16, True),   # 16 tokens (256 rows) per chunk
    (70, 128, 128, 96, 32, torch.float32, False),    # 8 tokens per chunk: half the routing waves idle
    (40, 128, 128, 64, 40, torch.float32, True),     # top_k > 32 is the routing's limit: rejected
])
def test_routed_call_matches_route_then_experts(cuda, tokens, hidden, inter, experts, top_k, ldtype, norm):
    """kq_moe_routed_block_fp8_experts (routing, histograms and token
    quantization in one launch; scan and scatter in one launch where the
    histogram table is small) against kq_moe_route_topk followed by
    kq_moe_block_fp8_experts: indices, weights and outputs equal bit for bit
    (the latter pair is checked against the oracle by the tests above), for
    every logits-per-lane form, chunk geometry and both scan forms."""
    banner(f"moe routed call tokens={tokens} E={experts} k={top_k} {ldtype} norm={norm}")
    pack = _pack(experts, hidden, inter, seed=tokens + experts, device=cuda)
    g = torch.Generator().manual_seed(tokens * 3 + top_k)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(tokens, experts, generator=g)
    logits[::5] = torch.round(logits[::5] * 2) / 2  # exact ties
    logits = logits.to(ldtype).to(cuda)
    if top_k > 32:
        with pytest.raises(ValueError, match="top_k <= 32"):
            pack.forward_logits(x, logits, top_k, norm)
        return
    idx, w = hmoe._route(logits, top_k, norm)
    expected = pack.forward(x, idx, w)
    out, idx2, w2 = pack.forward_logits(x, logits, top_k, norm)
    assert torch.equal(idx2, idx)
    assert torch.equal(w2.view(torch.int32), w.view(torch.int32))
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16))


@pytest.mark.parametrize("tokens,experts,top_k", [(333, 60, 6), (4096, 128, 8), (9000, 128, 8)])
def test_routed_call_fits_the_exact_workspace(cuda, tokens, experts, top_k):
    """The routed call's sort chunks (16 tokens where the chunk table fits
    the one-launch scan) outnumber the given-routing call's; both run in
    exactly kq_moe_workspace_size bytes (a buffer of that size with a guard
    region behind it that must stay untouched) and give the two-call bits."""
    banner(f"moe exact workspace tokens={tokens} E={experts} k={top_k}")
    hidden, inter = 128, 128
    pack = _pack(experts, hidden, inter, seed=tokens, device=cuda)
    g = torch.Generator().manual_seed(tokens + 3)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(tokens, experts, generator=g).to(cuda)
    idx, w = hmoe._route(logits, top_k, True)
    expected = pack.forward(x, idx, w)
    need = int(_native.library().kq_moe_workspace_size(tokens, hidden, inter, experts, top_k))
    guard = 1 << 16
    buf = torch.full((need + guard,), 0x5A, dtype=torch.uint8, device=cuda)
    out = torch.empty_like(x)
    idx2 = torch.empty(tokens, top_k, dtype=torch.int32, device=cuda)
    w2 = torch.empty(tokens, top_k, dtype=torch.float32, device=cuda)
    stream = _native.stream_handle(cuda)
    _native.call("kq_moe_routed_block_fp8_experts", logits.data_ptr(), _native.dtype_code(logits.dtype), 1,
                 x.data_ptr(), _native.dtype_code(x.dtype), tokens, hidden, inter, experts, top_k,
                 pack.w13.data_ptr(), pack.s13.data_ptr(), pack.w2.data_ptr(), pack.s2.data_ptr(),
                 idx2.data_ptr(), w2.data_ptr(), out.data_ptr(), buf.data_ptr(), need, stream)
    assert torch.equal(idx2, idx) and torch.equal(out.view(torch.int16), expected.view(torch.int16))
    out2 = torch.empty_like(x)
    _native.call("kq_moe_block_fp8_experts", x.data_ptr(), _native.dtype_code(x.dtype), tokens, hidden, inter,
                 experts, top_k, idx.data_ptr(), w.data_ptr(), pack.w13.data_ptr(), pack.s13.data_ptr(),
                 pack.w2.data_ptr(), pack.s2.data_ptr(), out2.data_ptr(), buf.data_ptr(), need, stream)
    assert torch.equal(out2.view(torch.int16), expected.view(torch.int16))
    assert bool((buf[need:] == 0x5A).all())
    with pytest.raises(RuntimeError, match="workspace"):
        _native.call("kq_moe_routed_block_fp8_experts", logits.data_ptr(), _native.dtype_code(logits.dtype), 1,
                     x.data_ptr(), _native.dtype_code(x.dtype), tokens, hidden, inter, experts, top_k,
                     pack.w13.data_ptr(), pack.s13.data_ptr(), pack.w2.data_ptr(), pack.s2.data_ptr(),
                     idx2.data_ptr(), w2.data_ptr(), out.data_ptr(), buf.data_ptr(), need - 256, stream)


def test_routed_call_graph_replays_match_eager(cuda):
    """The one-call block forward captured in a HIP graph: every replay (with
    eager calls of the same function between them) gives the eager bits."""
    pack = _pack(16, 256, 128, seed=7, device=cuda)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(300, 256, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(300, 16, generator=g).to(cuda)

    def step():
        return pack.forward_logits(x, logits, 4, True)[0]

    eager = step().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        step()
        torch.cuda.synchronize()


def test_row_tile_heights_agree_bit_for_bit(cuda):
    """1500 tokens x top-4 over 16 experts average 375 rows per expert, so the
    whole call runs 320-row tiles (several per expert, with tails); 128-token
    calls average 32 rows and run 256-row tiles.  A token's result does not
    depend on the tile it lands in, so both must agree bit for bit; a token
    sample is checked against the oracle."""
    tokens, top_k, experts = 1500, 4, 16
    banner(f"moe tile heights tokens={tokens} top_k={top_k} experts={experts}")
    pack = _pack(experts, 256, 256, seed=11, device=cuda)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(tokens, 256, generator=g).to(torch.bfloat16)
    idx = torch.argsort(torch.rand(tokens, experts, generator=g), dim=1)[:, :top_k].to(torch.int32)
    w = torch.softmax(torch.randn(tokens, top_k, generator=g), dim=1)
    xd, idxd, wd = x.to(cuda), idx.to(cuda), w.to(cuda)
    out = pack.forward(xd, idxd, wd)
    parts = torch.cat([pack.forward(xd[i:i + 128], idxd[i:i + 128], wd[i:i + 128])
                       for i in range(0, tokens, 128)])
    assert torch.equal(out, parts)
    sample = _covering_sample(idx.numpy(), experts, 96, seed=13)
    expected = _oracle_moe(pack, x, idx.numpy(), w.numpy(), tokens=sample)
    assert_moe_close(np32(out)[sample], expected, "bfloat16", label="tile heights", **_NARROW)


def test_fp16_experts_at_c5_widths_sampled_tokens(cuda):
    """fp16 activations through the 320-row tiles at C5's hidden / intermediate
    widths (K = 2048 for gate_up, 768 for down) and weight distribution
    (N(0, 0.02) before block quantization): 1024 tokens x top-8 over 32
    experts average 256 rows per expert; 160 tokens against the oracle, among
    them every expert's first row and the last row block of each row tile.
    fp16 outputs take 64 ulps (the relative width of bf16's 8): the e4m3
    re-quantization flips of the SwiGLU product move outputs by the same
    relative amount in either dtype, which at these widths is 8 or more fp16
    ulps for about 15% of the outputs (measured on gfx950); the relative-RMSE
    bound (5e-3) is unchanged."""
    tokens, hidden, inter, experts, top_k = 1024, 2048, 768, 32, 8
    banner("moe fp16 C5 widths")
    pack = _pack(experts, hidden, inter, seed=21, device=cuda, std=0.02)  # C5's weight distribution
    g = torch.Generator().manual_seed(22)
    x = torch.randn(tokens, hidden, generator=g).to(torch.float16)
    logits = torch.randn(tokens, experts, generator=g)
    idx, w = hmoe.route_logits(logits.to(cuda), top_k)
    out = pack.forward(x.to(cuda), idx, w)
    assert out.dtype == torch.float16
    sample = _covering_sample(idx.cpu().numpy(), experts, 160, seed=23)
    expected = _oracle_moe(pack, x, idx.cpu().numpy(), w.cpu().numpy(), tokens=sample)
    assert_moe_close(np32(out)[sample], expected, "float16", label="fp16 C5 widths", ulps=64.0)


def test_block_module_uses_grouped_path_and_matches_oracle(cuda):
    torch.manual_seed(2)
    block = hmoe.Qwen3BlockFp8MoeBlock(256, 128, 8, 2)
    hmoe.quantize_experts(block, torch.randn(8, 256, 256) * 0.05, torch.randn(8, 256, 128) * 0.05)
    with torch.no_grad():
        block.gate.weight.normal_(0, 0.1)
    block.gate.to(torch.bfloat16)
    x = torch.randn(2, 9, 256).to(torch.bfloat16)
    with torch.no_grad():
        block = block.to(cuda)
        pack = block._grouped_experts
        assert pack is not None and pack.w13.is_cuda
        gpu_out = block(x.to(cuda))
        idx, w = hmoe.route_logits(block.gate(x.to(cuda).reshape(-1, 256)), 2)
        two_calls = pack.forward(x.to(cuda).reshape(-1, 256), idx, w)
    assert gpu_out.shape == x.shape
    # the block routes inside the experts call: the same bits as route + experts
    assert torch.equal(gpu_out.reshape(-1, 256), two_calls)
    expected = _oracle_moe(pack, x.reshape(-1, 256), idx.cpu().numpy(), w.cpu().numpy())
    assert_moe_close(np32(gpu_out).reshape(-1, 256), expected, "bfloat16", label="block module", **_NARROW)


def test_c5_shape_sampled_tokens_and_determinism(cuda):
    banner("moe C5 full shape")
    wl = workloads.moe_layer(device=cuda)
    mod = wl.module
    out1 = mod(wl.x)
    out2 = mod(wl.x)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    idx, w = hmoe.route_logits(mod.logits, mod.top_k)
    counts = torch.bincount(idx.reshape(-1), minlength=128)
    assert int(counts.sum()) == 4096 * 8
    # every expert's first row and the last row block of its row tile, 320 tokens in all
    sample = _covering_sample(idx.cpu().numpy(), 128, 320, seed=0)
    assert len(sample) >= 256
    reached = np.unique(idx.cpu().numpy()[sample])
    assert reached.size == 128
    pack = hmoe.GroupedBlockFp8Experts.from_tensors(mod.w13, mod.s13, mod.w2, mod.s2)
    expected = _oracle_moe(pack, wl.x.cpu(), idx.cpu().numpy(), w.cpu().numpy(), tokens=sample)
    assert_moe_close(np32(out1)[sample], expected, "bfloat16", label=f"C5 {len(sample)} tokens")


def test_graph_replays_match_eager(cuda):
    pack = _pack(16, 256, 128, seed=5, device=cuda)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(64, 16, generator=g).to(cuda)

    def step():
        idx, w = hmoe._route(logits, 4, True)
        return pack.forward(x, idx, w)

    eager = step().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        step()
        torch.cuda.synchronize()


def test_rejects_bad_shapes(cuda):
    pack = _pack(4, 256, 128, seed=1, device=cuda)
    x = torch.randn(3, 256, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pack.forward(x, torch.zeros(3, 2, device=cuda, dtype=torch.int32), torch.ones(4, 2, device=cuda))
    with pytest.raises(ValueError):
        _native.call("kq_moe_route_topk", x.data_ptr(), 1, 3, 600, 2, 1, 0, 0,
                     torch.cuda.current_stream().cuda_stream)
    module = BlockFp8Linear(200, 256, bias=False).to(cuda)
    with pytest.raises(ValueError, match="in_features % 128"):
        module(torch.randn(2, 200, device=cuda, dtype=torch.bfloat16))


def test_factory_built_block_packs_its_experts_and_matches_oracle(cuda):
    """The reference's construction (moe.py:276-332): every routed expert
    projection through ``make_linear`` under the checkpoint's block-FP8
    quantization; the experts become BlockFp8Linear modules bound to the HIP
    forward, the block packs them (GroupedBlockFp8Experts.create) and the
    grouped call matches the oracle."""
    from kairyu_amd.quant.linear import LinearRole, linear_factory
    from kairyu_amd.quant.quant_config import detect_quantization

    banner("moe block through the factory")
    quant = detect_quantization({"quantization_config": {"quant_method": "fp8",
                                                         "weight_block_size": [128, 128]}})
    factory = linear_factory(quant, device=cuda, dtype=torch.bfloat16)
    block = hmoe.Qwen3BlockFp8MoeBlock(256, 128, 8, 2, linear_factory=factory, prefix="model.layers.1.mlp",
                                       layer_index=1)
    assert type(block.gate) is torch.nn.Linear                       # router stays dense
    assert block.gate.linear_selection.reason == "default-dense-role:moe_router"
    proj = block.experts[5].down_proj
    assert isinstance(proj, BlockFp8Linear) and proj._fused_forward is hip.block_fp8_linear_forward
    assert proj.linear_context.qualified_name == "model.layers.1.mlp.experts.5.down_proj"
    assert proj.linear_context.role is LinearRole.MLP_DOWN and proj.linear_context.expert_index == 5
    g = torch.Generator().manual_seed(17)
    hmoe.quantize_experts(block, torch.randn(8, 256, 256, generator=g) * 0.05,
                          torch.randn(8, 256, 128, generator=g) * 0.05)
    with torch.no_grad():
        block.gate.weight.normal_(0, 0.1, generator=g)
    block = block.to(cuda)
    block.gate.to(torch.bfloat16)
    pack = block._grouped_experts
    assert pack is not None and pack.w13.is_cuda and pack.is_current()
    x = torch.randn(37, 256, generator=g).to(torch.bfloat16).to(cuda)
    with torch.no_grad():
        out = block(x)
        idx, w = hmoe.route_logits(block.gate(x), 2)
    expected = _oracle_moe(pack, x.cpu(), idx.cpu().numpy(), w.cpu().numpy())
    assert_moe_close(np32(out), expected, "bfloat16", label="factory block", **_NARROW)
    # an expert projection on its own runs the bound dense block-FP8 kernel
    single = block.experts[3].up_proj(x)
    check_block_fp8(single, x, block.experts[3].up_proj, label="factory expert up_proj")


def test_single_route_with_empty_trailing_experts(cuda):
    """One token routed to expert 0 of 4 with weight 1 (reference
    tests/gpu/test_grouped_moe_gpu.py:133-146): experts 1..3 get no rows."""
    pack = _pack(4, 256, 128, seed=13, device=cuda)
    x = torch.randn(1, 256, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16).to(cuda)
    idx = torch.zeros(1, 1, dtype=torch.int64, device=cuda)
    w = torch.ones(1, 1, dtype=torch.float32, device=cuda)
    out = pack.forward(x, idx, w)
    expected = _oracle_moe(pack, x.cpu(), idx.cpu().numpy(), w.cpu().numpy())
    assert_moe_close(np32(out), expected, "bfloat16", label="single route", **_NARROW)
    # weight 1 on one slot: the combine is the expert's own output
    alone = moe.expert_forward(np32(x), _bits(pack.w13)[0], pack.s13[0].cpu().numpy(),
                               _bits(pack.w2)[0], pack.s2[0].cpu().numpy())
    assert np.array_equal(expected, alone)


def test_empty_input_preserves_shape(cuda):
    """No tokens (reference tests/gpu/test_grouped_moe_gpu.py:148-158): the
    output keeps the [0, H] shape and nothing is launched."""
    pack = _pack(4, 256, 128, seed=14, device=cuda)
    x = torch.empty(0, 256, device=cuda, dtype=torch.bfloat16)
    out = pack.forward(x, torch.empty(0, 2, dtype=torch.int64, device=cuda),
                       torch.empty(0, 2, dtype=torch.float32, device=cuda))
    assert out.shape == x.shape and out.dtype == x.dtype
    block = hmoe.Qwen3BlockFp8MoeBlock(256, 128, 4, 2).to(cuda)
    block.gate.to(torch.bfloat16)
    with torch.no_grad():
        assert block(torch.empty(3, 0, 256, device=cuda, dtype=torch.bfloat16)).shape == (3, 0, 256)


def test_grouped_path_has_no_host_synchronization(cuda):
    """The routed-expert call issues no host-synchronizing ops (reference
    tests/gpu/test_grouped_moe_gpu.py:87-130 asserts the same of its
    grouped path): no nonzero / unique / item."""
    pack = _pack(8, 256, 128, seed=15, device=cuda)
    g = torch.Generator().manual_seed(15)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(64, 8, generator=g).to(cuda)
    idx, w = hmoe._route(logits, 2, True)
    pack.forward(x, idx, w)
    torch.cuda.synchronize()
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        idx, w = hmoe._route(logits, 2, True)
        pack.forward(x, idx, w)
    keys = {event.key for event in prof.key_averages()}
    assert "aten::_local_scalar_dense" not in keys and "aten::nonzero" not in keys
    assert not any("unique" in key for key in keys)
    assert not any("synchronize" in key.lower() for key in keys)
