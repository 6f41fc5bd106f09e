"""Seeded synthetic workloads for the BASELINE configurations.

Each builder returns ready-to-run quantized modules (the package's own
``AwqLinear`` / ``GptqLinear`` / ``Fp8Linear`` / ``Int8Linear``) and
activations, generated with ``torch.Generator`` on the requested device, plus
the algorithmic byte / FLOP counts the roofline uses.  No checkpoint or
dataset is involved (there is no network); shapes and distributions follow
the configuration text.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from kairyu_amd.quant import awq as awq_format
from kairyu_amd.quant import gptq as gptq_format
from kairyu_amd.quant.fp8 import quantize_fp8
from kairyu_amd.quant.int8 import quantize_int8_weight
from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear


@dataclass
class Workload:
    name: str
    module: torch.nn.Module
    x: torch.Tensor
    bytes: int
    flops: int
    bound: str  # "hbm" | "mfma"
    extra: dict = field(default_factory=dict)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _uniform(shape, lo, hi, g, device, dtype=torch.float32):
    return (torch.rand(shape, generator=g, device=device) * (hi - lo) + lo).to(dtype)


def awq_layer(m: int = 16, n: int = 4096, k: int = 4096, group: int = 128, seed: int = 0,
              device="cuda", x_dtype=torch.float16) -> Workload:
    """C1: AWQ W4A16, asymmetric int4, q,z ~ U{0..15}, scales ~ U(0.002, 0.02)."""

    g = _gen(device, seed)
    q = torch.randint(0, 16, (k, n), generator=g, device=device, dtype=torch.int32)
    z = torch.randint(0, 16, (k // group, n), generator=g, device=device, dtype=torch.int32)
    scales = _uniform((k // group, n), 0.002, 0.02, g, device, torch.float16)
    x = torch.randn((m, k), generator=g, device=device).to(x_dtype)
    module = AwqLinear(k, n, bias=False, group_size=group).to(device)
    module.qweight.copy_(awq_format.pack_awq(q))
    module.qzeros.copy_(awq_format.pack_awq(z))
    module.scales.copy_(scales)
    nbytes = k * n // 2 + (k // group) * (n // 8) * 4 + (k // group) * n * 2 + m * k * 2 + m * n * 2
    return Workload(f"awq_w4a16_m{m}_n{n}_k{k}_g{group}", module, x, nbytes, 2 * m * n * k,
                    "hbm" if m <= 64 else "mfma")


def gptq_layer(m: int = 16, n: int = 28672, k: int = 4096, group: int = 128, seed: int = 0,
               device="cuda", x_dtype=torch.float16, act_order: bool = True) -> Workload:
    """C2: GPTQ W4A16 symmetric (stored zeros 7, z = 8), act-order g_idx =
    randperm(K) // group, scales ~ U(0.001, 0.01)."""

    g = _gen(device, seed)
    q = torch.randint(0, 16, (k, n), generator=g, device=device, dtype=torch.int32)
    groups = -(-k // group)
    scales = _uniform((groups, n), 0.001, 0.01, g, device, torch.float16)
    if act_order:
        g_idx = (torch.randperm(k, generator=g, device=device) // group).to(torch.int32)
    else:
        g_idx = (torch.arange(k, device=device) // group).to(torch.int32)
    x = torch.randn((m, k), generator=g, device=device).to(x_dtype)
    module = GptqLinear(k, n, bias=False, group_size=group).to(device)
    module.qweight.copy_(gptq_format.pack_gptq_rows(q))
    module.qzeros.copy_(
        gptq_format.pack_gptq_cols(torch.full((groups, n), 7, dtype=torch.int32)).to(device)
    )
    module.scales.copy_(scales)
    module.g_idx.copy_(g_idx)
    nbytes = (k * n // 2 + groups * (n // 8) * 4 + groups * n * 2 + 4 * k + m * k * 2 + m * n * 2)
    return Workload(f"gptq_w4a16_actorder_m{m}_n{n}_k{k}_g{group}", module, x, nbytes,
                    2 * m * n * k, "hbm" if m <= 64 else "mfma")


def fp8_layer(m: int = 16, n: int = 4096, k: int = 14336, seed: int = 0, device="cuda",
              x_dtype=torch.bfloat16) -> Workload:
    """C3: FP8 e4m3 W8A8, W ~ N(0, 0.02) per-channel; x ~ N(0,1) with exactly
    floor(0.01*M*K) (at least one) seeded outliers x20; dynamic per-token quant."""

    g = _gen(device, seed)
    w = torch.randn((n, k), generator=g, device=device) * 0.02
    qw, ws = quantize_fp8(w, per_channel=True)
    del w
    x = torch.randn((m, k), generator=g, device=device)
    count = max(1, (m * k) // 100)
    flat_idx = torch.randperm(m * k, generator=g, device=device)[:count]
    x.view(-1)[flat_idx] *= 20.0
    module = Fp8Linear(k, n, bias=False).to(device)
    module.weight.copy_(qw)
    module.weight_scale.copy_(ws)
    nbytes = n * k + 4 * n + 2 * m * k + 2 * m * n + 4 * m
    return Workload(f"fp8_w8a8_m{m}_n{n}_k{k}", module, x.to(x_dtype), nbytes, 2 * m * n * k,
                    "hbm" if m <= 64 else "mfma")


def int8_layer(m: int = 16, n: int = 18944, k: int = 3584, seed: int = 0, device="cuda",
               x_dtype=torch.bfloat16) -> Workload:
    """C4: INT8 W8A8 SmoothQuant-style, W ~ N(0, 0.02) per-channel int8; x ~ N(0,1)."""

    g = _gen(device, seed)
    w = torch.randn((n, k), generator=g, device=device) * 0.02
    qw, ws = quantize_int8_weight(w)
    del w
    x = torch.randn((m, k), generator=g, device=device).to(x_dtype)
    module = Int8Linear(k, n, bias=False).to(device)
    module.weight.copy_(qw)
    module.weight_scale.copy_(ws)
    nbytes = n * k + 4 * n + 2 * m * k + 2 * m * n + 4 * m
    return Workload(f"int8_w8a8_m{m}_n{n}_k{k}", module, x, nbytes, 2 * m * n * k,
                    "hbm" if m <= 64 else "mfma")


def reference_microbench_layer(scheme: str, m: int, n: int = 4096, k: int = 4096, seed: int = 205,
                               device="cuda") -> Workload:
    """The reference's own microbenchmark setup
    (verification/l1/performance/quant_gemm_bench.py:184-196): torch seed 205,
    weight ``randn(n, k)`` quantized by the format's quantizer (FP8 per
    channel, INT8 per channel, AWQ / GPTQ groups of 128 along K), x
    ``randn(m, k)`` in bf16 on the device (drawn after the weight, from the
    global generator as the reference does)."""

    from kairyu_amd.quant.awq import quantize_awq
    from kairyu_amd.quant.gptq import quantize_gptq

    torch.manual_seed(seed)
    weight = torch.randn(n, k)
    if scheme == "fp8":
        module = Fp8Linear(k, n, bias=False)
        qw, ws = quantize_fp8(weight)
        module.weight.copy_(qw)
        module.weight_scale.copy_(ws)
    elif scheme == "int8":
        module = Int8Linear(k, n, bias=False)
        qw, ws = quantize_int8_weight(weight)
        module.weight.copy_(qw)
        module.weight_scale.copy_(ws)
    elif scheme == "awq":
        module = AwqLinear(k, n, bias=False, group_size=128)
        for name, t in zip(("qweight", "qzeros", "scales"), quantize_awq(weight, group_size=128)):
            getattr(module, name).copy_(t)
    elif scheme == "gptq":
        module = GptqLinear(k, n, bias=False, group_size=128)
        for name, t in zip(("qweight", "qzeros", "scales", "g_idx"), quantize_gptq(weight, group_size=128)):
            getattr(module, name).copy_(t)
    else:
        raise ValueError(f"unknown scheme {scheme!r}")
    module = module.to(device)
    x = torch.randn(m, k, device=device, dtype=torch.bfloat16)
    w4 = scheme in ("awq", "gptq")
    groups = k // 128
    nbytes = (k * n // 2 + groups * (n // 8) * 4 + groups * n * 2 if w4 else n * k + 4 * n) + m * k * 2 + m * n * 2
    return Workload(f"reference_microbench_{scheme}_m{m}_n{n}_k{k}", module, x, nbytes, 2 * m * n * k,
                    "hbm" if m <= 64 else "mfma")


def replicas(workload: Workload, copies: int) -> list[torch.nn.Module]:
    """Independent copies of a workload's module (distinct HBM allocations), used
    to rotate weights so repeated calls cannot be served from the 256 MB MALL."""

    mods = [workload.module]
    for _ in range(copies - 1):
        clone = type(workload.module).__new__(type(workload.module))
        clone.__dict__ = dict(workload.module.__dict__)
        clone._buffers = {name: t.clone() for name, t in workload.module._buffers.items()}
        clone._parameters = dict(workload.module._parameters)
        clone._modules = dict(workload.module._modules)
        clone.__dict__.pop("_kq_gptq_operands", None)
        clone.__dict__.pop("_kq_awq_operands", None)
        mods.append(clone)
    return mods


class MoeFromLogits(torch.nn.Module):
    """C5 step on given router logits (the router GEMM is excluded): Qwen3
    top-k routing, then the block-FP8 experts with the fp32 slot-order
    combine."""

    def __init__(self, w13, s13, w2, s2, logits, top_k: int, norm_topk_prob: bool = True):
        super().__init__()
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        for name, t in (("w13", w13), ("s13", s13), ("w2", w2), ("s2", s2), ("logits", logits)):
            self.register_buffer(name, t)

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        from kairyu_amd import moe

        pack = moe.GroupedBlockFp8Experts.from_tensors(self.w13, self.s13, self.w2, self.s2)
        out, _, _ = pack.forward_logits(hidden, self.logits, self.top_k, self.norm_topk_prob)
        return out


def moe_layer(tokens: int = 4096, hidden: int = 2048, inter: int = 768, experts: int = 128,
              top_k: int = 8, seed: int = 0, device="cuda", norm_topk_prob: bool = True,
              x_dtype=torch.bfloat16) -> Workload:
    """C5: Qwen3-MoE-like block-FP8 experts, E=128, H=2048, I=768; gate_up
    [E, 1536, 2048] (gate rows first) and down [E, 2048, 768] ~ N(0, 0.02)
    quantized per 128x128 block; hidden bf16 ~ N(0,1) [4096, 2048]; router
    logits ~ N(0,1) [4096, 128], top-8."""

    from kairyu_amd.quant.block_fp8 import quantize_block_fp8

    g = _gen(device, seed)
    w13 = torch.empty((experts, 2 * inter, hidden), dtype=torch.float8_e4m3fn, device=device)
    s13 = torch.empty((experts, 2 * inter // 128, hidden // 128), dtype=torch.float32, device=device)
    w2 = torch.empty((experts, hidden, inter), dtype=torch.float8_e4m3fn, device=device)
    s2 = torch.empty((experts, hidden // 128, inter // 128), dtype=torch.float32, device=device)
    for e in range(0, experts, 16):
        sl = slice(e, min(experts, e + 16))
        count = sl.stop - sl.start
        q, s = quantize_block_fp8(torch.randn((count, 2 * inter, hidden), generator=g, device=device) * 0.02)
        w13[sl], s13[sl] = q, s
        q, s = quantize_block_fp8(torch.randn((count, hidden, inter), generator=g, device=device) * 0.02)
        w2[sl], s2[sl] = q, s
    x = torch.randn((tokens, hidden), generator=g, device=device).to(x_dtype)
    logits = torch.randn((tokens, experts), generator=g, device=device)
    module = MoeFromLogits(w13, s13, w2, s2, logits, top_k, norm_topk_prob)
    weight_bytes = experts * (2 * inter * hidden + hidden * inter)
    scale_bytes = experts * ((2 * inter // 128) * (hidden // 128) + (hidden // 128) * (inter // 128)) * 4
    nbytes = weight_bytes + scale_bytes + 2 * tokens * hidden * 2
    flops = 2 * tokens * top_k * (2 * inter * hidden + hidden * inter)
    return Workload(f"moe_block_fp8_t{tokens}_h{hidden}_i{inter}_e{experts}_k{top_k}", module, x,
                    nbytes, flops, "hbm")
