"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (``value``): GPTQ act-order W4A16 (N=28672,
K=4096, group 128) at decode size M=16, as whole-op HBM throughput in GB/s of
algorithmic bytes.  One step = one forward of the quantized linear on one
batch; weights rotate over enough distinct HBM copies (> 256 MB MALL) that no
step is served from the Infinity Cache.  `--steps` steps are captured in one
HIP graph; each timing sample replays it back to back for at least 200 steps
(HIP events on the stream they run on, one untimed replay queued first), and
every time reported is the median of 7 samples, with their spread
(``timing``).

``roofline`` describes the headline's dominant kernel alone: the decode
GEMV's algorithmic bytes per launch over its per-launch time, timed live with
HIP events on its own captured launches (x gathered once up front).

``sweep`` reports every BASELINE configuration (C1-C4 over their M values,
C5) and decode (M = 1, 16) at the other projection shapes of Llama-3-8B and
Qwen2-7B for AWQ, GPTQ act-order and FP8, each row with
  * ``op``: the whole module call (activation quantization / act-order gather
    included) -- GB/s, TFLOPS and both roofline fractions;
  * ``gemm``: the dominant GEMM entry alone on pre-processed activations
    (gathered fp16 x, quantized int8 / e4m3 rows), its algorithmic bytes or
    FLOPs per launch over the per-launch time (none for C5, whose kernels are
    split in ``profiles/``);
  * ``vendor_gemm`` (W8A8 prefill rows, M > 64): the vendor library
    (hipBLASLt through torch) on the same quantized operands and weight
    copies, with the ratio of its time to the ``gemm`` time;
  * ``cpu_baseline`` and ``parity`` (unless ``--no-cpu``): the repo's CPU
    restatement of the reference path timed on a bounded sample of the row's
    workload on this host's cores, and the device output on the same sample
    judged against the oracle with the test suite's criteria
    (``oracle.parity``).
``context`` holds the reference microbenchmark's own setup (N = K = 4096, M
in {1, 128}, bf16, seed 205, four formats) timed its way and this bench's
way, next to its published numbers on its own GPU (``--no-context`` skips).
The top-level ``cpu_baseline`` is the headline row's.  ``peaks`` holds the
box's measured ceilings (streaming read, MFMA loop per dtype; see
``measure_peaks``), and every roofline entry gives its fraction of the
measured ceiling (``frac_of_measured_peak``) next to the vendor one.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep]
                       [--no-cpu] [--no-headline] [--no-peaks] [--only SUBSTRING[|SUBSTRING]]
       python bench.py --peaks             (measured ceilings only)
       python bench.py --floors            (empty kernel per graph step)
       python bench.py --copy-calibration  (256 MiB copies for counter scaling)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp16": 2500.0, "fp8": 5000.0, "int8": 5000.0}
MALL_BYTES = 256 * 1024 * 1024


def _weight_bytes(module) -> int:
    return sum(t.numel() * t.element_size() for t in module.buffers(recurse=False))


def _copies(module) -> int:
    return min(64, max(1, math.ceil(1.25 * MALL_BYTES / max(1, _weight_bytes(module)))))


def clock_warmup(seconds: float = 1.0) -> None:
    """Run dense GEMMs for about `seconds` so clocks and power state settle
    before the first timed region."""

    import torch

    a = torch.randn(8192, 8192, device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            a = (a @ a).clamp_(-1.0, 1.0)
        torch.cuda.synchronize()
    del a


def _timed_replays(graph, steps: int, samples: int = 7, min_launches: int = 200,
                   settle_s: float = 0.3) -> dict:
    """ms per captured step: the median over `samples` timed samples, each of
    enough back-to-back replays of the `steps`-launch graph for at least
    `min_launches` launches, whatever `steps` is.  HIP events on the replaying
    stream bracket each sample, and one untimed replay is queued before the
    start event so the GPU is already busy when it fires (the host's first
    submission is not timed).  Untimed replays first, for at least `settle_s`
    seconds: the GPU idles while the host builds a workload and its graph, and
    its clocks need that long under load to return to their steady state.
    Returns {"ms", "samples", "launches_per_sample", "spread"} with spread =
    (slowest - fastest sample) / median."""

    import torch

    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < settle_s:
        graph.replay()
        torch.cuda.synchronize()
    reps = max(1, math.ceil(min_launches / steps))
    times = []
    for _ in range(samples):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        graph.replay()  # untimed: keeps the queue busy across the start event
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / (reps * steps))
    times.sort()
    median = times[len(times) // 2]
    return {"ms": median, "samples": samples, "launches_per_sample": reps * steps,
            "spread": round((times[-1] - times[0]) / median, 4) if median > 0 else 0.0}


def _graph_ms(launch, copies: int, steps: int, warmup: int = 0, stats: dict | None = None) -> float:
    """ms per launch of `launch(i)` (i = step index, rotating over `copies`
    operand sets), captured `steps` times in one graph (timing statistics
    into `stats` when given)."""

    import torch

    for i in range(max(warmup, copies)):
        launch(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(copies):
            launch(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            launch(i)
    timing = _timed_replays(graph, steps)
    if stats is not None:
        stats.update(timing)
    del graph
    return timing["ms"]


def measure(workload, steps: int, warmup: int) -> dict:
    """Whole module call, weights rotating over distinct copies."""

    from kairyu_amd import workloads

    copies = _copies(workload.module)
    mods = workloads.replicas(workload, copies)
    x = workload.x
    stats: dict = {}
    ms = _graph_ms(lambda i: mods[i % copies](x), copies, steps, warmup, stats)
    return {"ms": ms, "gbps": workload.bytes / (ms * 1e-3) / 1e9,
            "tflops": workload.flops / (ms * 1e-3) / 1e12, "copies": copies,
            "timing": {k: stats[k] for k in ("samples", "launches_per_sample", "spread")}}


def gemm_launcher(workload, copies: int):
    """(launch(i), algorithmic bytes, flops, kernel description) of the
    workload's dominant GEMM entry alone, on pre-processed activations, or
    None for workloads without a single dominant GEMM entry (MoE)."""

    import torch

    from kairyu_amd import _native, workloads
    from kairyu_amd.kernels import quant_gemm_hip as hip
    from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear

    module, x = workload.module, workload.x
    if not isinstance(module, (AwqLinear, GptqLinear, Fp8Linear, Int8Linear)):
        return None
    device = x.device
    m, k = x.shape
    n = module.out_features
    mods = workloads.replicas(workload, copies)
    if isinstance(module, (AwqLinear, GptqLinear)):
        group = module.group_size
        groups = -(-k // group)
        if isinstance(module, GptqLinear):
            ops = [hip._gptq_operands(mod, device) for mod in mods]
            mode, _, perm = ops[0]
            x16 = x[:, perm.long()].contiguous() if mode == hip.GIDX_PERMUTED else x
            operands = [(t.tiles, t.zeros, t.zero_offset, mod.scales) for mod, (_, t, _) in zip(mods, ops)]
        else:
            ops = [hip._awq_operands(mod, device) for mod in mods]
            x16 = x
            operands = [(t.tiles, t.zeros, t.zero_offset, mod.scales) for mod, t in zip(mods, ops)]
        out = torch.empty((m, n), device=device, dtype=x.dtype)
        ws = _native.workspace(device, int(_native.library().kq_w4a16_workspace_size(m, n, k, 0)))

        def launch(i):
            tiles, zeros, zoff, scales = operands[i % copies]
            _native.call("kq_w4a16_tiled_gemm", x16.data_ptr(), _native.dtype_code(x16.dtype),
                         tiles.data_ptr(), _native.ptr(zeros), zoff, scales.data_ptr(), None, None,
                         _native.DTYPE_NONE, out.data_ptr(), m, n, k, group, ws.data_ptr(), ws.numel(),
                         _native.stream_handle(device))

        nbytes = k * n // 2 + groups * (n // 8) * 4 + groups * n * 2 + m * k * 2 + m * n * 2
        kernel = ("w4a16_gemv_kernel (M <= 16 decode GEMV)" if m <= 16
                  else "w4a16_prefill_kernel (+ its fp16 staging pass)")
        return launch, nbytes, 2 * m * n * k, kernel
    fp8 = isinstance(module, Fp8Linear)
    xq, xs = hip._quantize_activation(x, torch.float8_e4m3fn if fp8 else torch.int8,
                                      448.0 if fp8 else 127.0)
    wscales = [hip._f32(mod.weight_scale) for mod in mods]
    out = torch.empty((m, n), device=device, dtype=x.dtype)
    ws = _native.workspace(device, int(_native.library().kq_w8a8_workspace_size(m, n, k)))

    def launch(i):
        mod, wsc = mods[i % copies], wscales[i % copies]
        if fp8:
            _native.call("kq_w8a8_fp8_gemm", xq.data_ptr(), xs.data_ptr(), mod.weight.data_ptr(),
                         wsc.data_ptr(), int(wsc.numel() != 1), None, _native.DTYPE_NONE,
                         out.data_ptr(), _native.dtype_code(x.dtype), m, n, k, ws.data_ptr(),
                         ws.numel(), _native.stream_handle(device))
        else:
            _native.call("kq_w8a8_i8_gemm", xq.data_ptr(), xs.data_ptr(), mod.weight.data_ptr(),
                         wsc.data_ptr(), None, _native.DTYPE_NONE, out.data_ptr(),
                         _native.dtype_code(x.dtype), None, m, n, k, ws.data_ptr(), ws.numel(),
                         _native.stream_handle(device))

    nbytes = n * k + 4 * n + m * k + 4 * m + 2 * m * n
    # the launcher's dispatch in kq_w8a8.hip: decode kernel for M <= 16 with
    # K % 128 == 0, skinny kernel up to M = 64, tile engine above
    if m <= 16 and k % 128 == 0:
        kernel = "w8a8_decode_kernel"
    elif m <= 64:
        kernel = "w8a8_skinny_kernel (+ split-K reduce when used)"
    else:
        kernel = "tile_gemm_kernel (+ split-K reduce when used)"
    return launch, nbytes, 2 * m * n * k, kernel


def measure_gemm(workload, steps: int, dtype: str) -> dict | None:
    copies = _copies(workload.module)
    spec = gemm_launcher(workload, copies)
    if spec is None:
        return None
    launch, nbytes, flops, kernel = spec
    stats: dict = {}
    ms = _graph_ms(launch, copies, steps, stats=stats)
    gbps = nbytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    hbm = workload.bound == "hbm"
    achieved = gbps if hbm else tflops
    peak = HBM_PEAK_GBS if hbm else MFMA_PEAK_TFLOPS[dtype]
    return {"kernel": kernel, "us": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
            "flops_per_launch": flops, "bound": workload.bound, "achieved": round(achieved, 1),
            "unit": "GB/s" if hbm else "TFLOP/s", "peak": peak, "frac": round(achieved / peak, 4),
            "timing": {k: stats[k] for k in ("samples", "launches_per_sample", "spread")}}


def vendor_gemm(workload, steps: int) -> dict | None:
    """The vendor library on the same quantized operands, for the W8A8
    prefill rows (M > 64): hipBLASLt through torch._scaled_mm (e4m3 x e4m3,
    fp32 row scales x fp32 column scales, bf16 out: the same epilogue) or
    torch._int_mm (int8 x int8 -> int32, no scale epilogue).  Timed eagerly
    with events over `steps` calls rotating the same weight copies as
    measure_gemm (library calls stay out of graph capture)."""

    import torch

    from kairyu_amd import workloads
    from kairyu_amd.kernels import quant_gemm_hip as hip
    from kairyu_amd.quant.linear import Fp8Linear, Int8Linear

    module, x = workload.module, workload.x
    m, k = x.shape
    if not isinstance(module, (Fp8Linear, Int8Linear)) or m <= 64:
        return None
    n = module.out_features
    copies = _copies(module)
    mods = workloads.replicas(workload, copies)
    fp8 = isinstance(module, Fp8Linear)
    xq, xs = hip._quantize_activation(x, torch.float8_e4m3fn if fp8 else torch.int8,
                                      448.0 if fp8 else 127.0)
    if fp8:
        sa = xs.reshape(m, 1).float()
        sbs = [hip._f32(mod.weight_scale).reshape(1, -1).expand(1, n).contiguous() for mod in mods]
        call = lambda i: torch._scaled_mm(xq, mods[i % copies].weight.t(), scale_a=sa,  # noqa: E731
                                          scale_b=sbs[i % copies], out_dtype=x.dtype)
        lib = "hipBLASLt via torch._scaled_mm (row-wise fp32 scales, bf16 out)"
    else:
        call = lambda i: torch._int_mm(xq, mods[i % copies].weight.t())  # noqa: E731
        lib = "hipBLASLt via torch._int_mm (int32 out, no scale epilogue)"
    try:
        for i in range(max(5, copies)):
            call(i)
        torch.cuda.synchronize()
    except RuntimeError as exc:  # an older torch without row-wise scaling
        return {"library": lib, "error": str(exc)[:200]}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        call(i)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return {"library": lib, "us": round(ms * 1e3, 3),
            "achieved": round(2 * m * n * k / (ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s"}


# ------------------------------------------------------------ CPU baselines
def _blas_threads() -> int:
    from threadpoolctl import threadpool_info

    return int(max((p.get("num_threads", 1) for p in threadpool_info()), default=1))


def _median_time(fn, target_s: float, max_runs: int = 20) -> tuple[float, int]:
    fn()  # warm up
    times = []
    deadline = time.perf_counter() + target_s
    while len(times) < 3 or (time.perf_counter() < deadline and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(sorted(times)[len(times) // 2]), len(times)


def _np(t):
    import torch

    return t.detach().to("cpu", torch.float32).numpy()


def _bits_np(t):
    import torch

    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def cpu_row(name: str, workload, gpu_out, target_s: float = 2.0) -> tuple[dict, dict]:
    """(cpu_baseline, parity) of one sweep row: the oracle's port of the
    reference CPU path timed on a bounded sample of the row's workload, and
    the device output judged on a sample against the oracle's exact path."""

    import numpy as np

    from kairyu_amd.quant.linear import AwqLinear, Fp8Linear, GptqLinear, Int8Linear
    from oracle import linear as olinear
    from oracle import moe as omoe
    from oracle import parity
    from oracle.numerics import e4m3_decode

    module, x = workload.module, workload.x
    m, k = x.shape
    out_np = _np(gpu_out)
    cores = _blas_threads()
    dt = {"torch.float16": "float16", "torch.bfloat16": "bfloat16"}[str(x.dtype)]
    if isinstance(module, (AwqLinear, GptqLinear)):
        n = module.out_features
        cols = min(n, 7168)
        xs = _np(x)
        qw, qz, sc = module.qweight.cpu().numpy(), module.qzeros.cpu().numpy(), _np(module.scales)
        groups = sc.shape[0]
        if isinstance(module, GptqLinear):
            gi = module.g_idx.cpu().numpy()
            run = (lambda: olinear.gptq_forward_fast(xs, qw[:, :cols], qz[:, :cols // 8], sc[:, :cols], gi, dt))
            ref = (lambda c0, c1: olinear.gptq_reference(xs, qw[:, c0:c1], qz[:, c0 // 8:c1 // 8],
                                                         sc[:, c0:c1], gi, dt))
        else:
            g = module.group_size
            run = (lambda: olinear.awq_forward_fast(xs, qw[:, :cols // 8], qz[:, :cols // 8], sc[:, :cols], g, dt))
            ref = (lambda c0, c1: olinear.awq_reference(xs, qw[:, c0 // 8:c1 // 8], qz[:, c0 // 8:c1 // 8],
                                                        sc[:, c0:c1], g, dt))
        med, runs = _median_time(run, target_s)
        scale = n / cols
        nbytes = workload.bytes
        value = nbytes / (med * scale) / 1e9
        cpu = {"value": round(value, 3), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": (f"oracle.linear.{'gptq' if isinstance(module, GptqLinear) else 'awq'}_forward_fast "
                          f"(numpy dequantize -> fp16 weight -> fp32 BLAS) on M={m} K={k} N={cols} of {n}, "
                          f"median of {runs} runs = {med * 1e3:.1f} ms, scaled by N; {groups} groups")}
        checks = []
        for c0 in sorted({0, (n // 2 - 256) // 8 * 8, n - 512}):
            pre, terms = ref(c0, c0 + 512)
            checks.append(parity.ulp_check(out_np[:, c0:c0 + 512], pre, dt,
                                           parity.fp16_mfma_slack(terms, k)))
        par = _summarize(checks, f"columns 0:512, middle 512, last 512 of all {m} rows")
        return cpu, par
    if isinstance(module, (Fp8Linear, Int8Linear)):
        n = module.out_features
        rows = np.arange(m) if m <= 32 else np.unique(np.r_[0:16, m - 16:m])
        xs = _np(x)[rows]
        w_np = module.weight.cpu()
        wscale = _np(module.weight_scale)
        if isinstance(module, Fp8Linear):
            from oracle import formats

            wb = _bits_np(w_np)
            t0 = time.perf_counter()
            wdec = e4m3_decode(wb)
            decode_s = time.perf_counter() - t0
            xb, xsc = formats.fp8_quantize_rows(xs)
            med, runs = _median_time(lambda: olinear.fp8_forward_fast(xb, xsc, wdec, wscale), target_s)
            total = decode_s + med * (m / len(rows))
            cpu = {"value": round(workload.flops / total / 1e12, 4) if m > 64 else
                   round(workload.bytes / total / 1e9, 3),
                   "unit": "TFLOP/s" if m > 64 else "GB/s", "cores": cores, "kind": "port",
                   "sample": (f"oracle.linear.fp8_forward_fast (fp32 BLAS of decoded e4m3) on {len(rows)} of "
                              f"{m} rows ({med * 1e3:.1f} ms, median of {runs}) + the weight decode "
                              f"({decode_s * 1e3:.0f} ms), extrapolated linearly in rows")}
            _, x_bits, x_scale, pre = olinear.fp8_forward(xs, wb, wscale)
            terms = olinear.fp8_abs_terms(x_bits, wb, x_scale, wscale)
            wsv = np.abs(wscale.astype(np.float64)).reshape(-1, 1)
            slack = parity.e4m3_mfma_slack(terms, k, np.abs(e4m3_decode(x_bits)) * x_scale,
                                           np.abs(wdec) * wsv)
            par = _summarize([parity.ulp_check(out_np[rows], pre, dt, slack)],
                             f"{len(rows)} rows (first and last 16) x all {n} columns")
            return cpu, par
        wq = w_np.numpy()
        run = lambda: olinear.int8_forward(xs, wq, wscale, None, out_dtype=dt)  # noqa: E731
        med, runs = _median_time(run, target_s, max_runs=5)
        total = med * (m / len(rows))
        cpu = {"value": round(workload.flops / total / 1e12, 4) if m > 64 else
               round(workload.bytes / total / 1e9, 3),
               "unit": "TOP/s" if m > 64 else "GB/s", "cores": cores, "kind": "port",
               "sample": (f"oracle.linear.int8_forward (exact int32 accumulation through fp64 BLAS) "
                          f"on {len(rows)} of {m} rows, median of {runs} = {med * 1e3:.1f} ms, "
                          f"extrapolated linearly in rows")}
        expected, *_ = run()
        same = bool(np.array_equal(out_np[rows].view(np.uint32), expected.astype(np.float32).view(np.uint32)))
        par = {"verdict": "pass" if same else "FAIL", "criterion": "bf16 output bit-exact",
               "sample": f"{len(rows)} rows x all {n} columns"}
        return cpu, par
    # MoE: the per-expert loop on a token sample (one timed run: the loop's
    # per-expert weight decode dominates and the result is deterministic)
    tokens = 16
    sel = np.random.default_rng(0).choice(m, size=tokens, replace=False)
    from kairyu_amd import moe as hmoe

    idx, w = hmoe.route_logits(module.logits, module.top_k, module.norm_topk_prob)
    args = (_np(x)[sel], idx.cpu().numpy()[sel], w.cpu().numpy()[sel], _bits_np(module.w13),
            module.s13.cpu().numpy(), _bits_np(module.w2), module.s2.cpu().numpy(), dt)
    t0 = time.perf_counter()
    expected = omoe.moe_forward(*args)
    elapsed = time.perf_counter() - t0
    total = elapsed * m / tokens
    cpu = {"value": round(workload.bytes / total / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
           "sample": (f"oracle.moe.moe_forward (per-expert loop, fp64 block sums) on {tokens} of {m} tokens "
                      f"({elapsed:.1f} s, one run), extrapolated linearly in tokens")}
    check = parity.moe_check(out_np[sel], expected, dt, min_col_rows=tokens)
    par = _summarize([check], f"{tokens} tokens x all {x.shape[1]} outputs", moe=True)
    return cpu, par


def _summarize(checks, sample: str, moe: bool = False) -> dict:
    ok = all(c["ok"] for c in checks)
    out = {"verdict": "pass" if ok else "FAIL",
           "criterion": ("per-element atol 2e-2 + rtol 1e-2, normwise 1e-2, per-row RMSE and "
                         "statistical (oracle.parity.moe_check)" if moe else
                         "per-element ulp + MFMA slack, rel-RMSE (oracle.parity.ulp_check)"),
           "sample": sample,
           "normwise_max": max(c.get("normwise_max", 0.0) for c in checks),
           "rel_rmse": max(c.get("rel_rmse", 0.0) for c in checks)}
    if not moe:
        out["max_ulp"] = round(max(c.get("max_ulp", 0.0) for c in checks), 3)
    if not ok:
        out["why"] = "; ".join(c.get("why", "") for c in checks if not c["ok"])
    return out


def cpu_baseline(target_seconds: float = 12.0) -> dict:
    """Time the oracle's GPTQ act-order forward on a column slice of the
    headline workload (M=16, K=4096, N=7168 of 28672) on this host."""

    import numpy as np

    from oracle import formats
    from oracle import linear as olinear

    rng = np.random.default_rng(0)
    m, k, n, group = 16, 4096, 7168, 128
    q = rng.integers(0, 16, size=(k, n))
    qweight = formats.gptq_pack_rows(q)
    qzeros = formats.gptq_pack_cols(np.full((k // group, n), 7))
    scales = rng.uniform(0.001, 0.01, size=(k // group, n)).astype(np.float16)
    g_idx = (rng.permutation(k) // group).astype(np.int32)
    x = rng.standard_normal((m, k)).astype(np.float16)
    nbytes = k * n // 2 + (k // group) * (n // 8) * 4 + (k // group) * n * 2 + 4 * k + m * k * 2 + m * n * 2
    med, runs = _median_time(lambda: olinear.gptq_forward_fast(x, qweight, qzeros, scales, g_idx, "float16"),
                             target_seconds, max_runs=50)
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": _blas_threads(),
        "kind": "port",
        "sample": (f"oracle.linear.gptq_forward_fast (numpy dequantize -> fp16 weight -> fp32 BLAS "
                   f"matmul) on M=16 K=4096 N=7168 (1/4 of C2's columns), median of {runs} "
                   f"runs = {med * 1e3:.1f} ms; host os.cpu_count()={os.cpu_count()}"),
    }


def sweep_entries():
    from kairyu_amd import workloads as W

    entries = [("C1 AWQ W4A16 N=K=4096 g128", "fp16", lambda: W.awq_layer(m=16))]
    for m in (1, 4, 16, 64, 512):
        entries.append((f"C2 GPTQ act-order W4A16 N=28672 K=4096 g128 M={m}", "fp16",
                        lambda m=m: W.gptq_layer(m=m)))
    for m in (1, 16, 2048, 8192):
        entries.append((f"C3 FP8 W8A8 N=4096 K=14336 M={m}", "fp8", lambda m=m: W.fp8_layer(m=m)))
    for m in (16, 4096):
        entries.append((f"C4 INT8 W8A8 N=18944 K=3584 M={m}", "int8", lambda m=m: W.int8_layer(m=m)))
    entries.append(("C5 block-FP8 MoE E=128 H=2048 I=768 T=4096 top8", "fp8", lambda: W.moe_layer()))
    # decode at the other projection shapes of the models north_star names
    # (kairyu/models/layers.py:212-241, attention.py:51-94)
    for label, n, k in DECODE_SHAPES:
        for m in (1, 16):
            entries.append((f"{label} AWQ W4A16 N={n} K={k} M={m}", "fp16",
                            lambda m=m, n=n, k=k: W.awq_layer(m=m, n=n, k=k)))
            entries.append((f"{label} GPTQ act-order W4A16 N={n} K={k} M={m}", "fp16",
                            lambda m=m, n=n, k=k: W.gptq_layer(m=m, n=n, k=k)))
            entries.append((f"{label} FP8 W8A8 N={n} K={k} M={m}", "fp8",
                            lambda m=m, n=n, k=k: W.fp8_layer(m=m, n=n, k=k)))
    # batched decode (M = 17..64): the skinny W8A8 GEMM with grouped column tiles
    entries.append(("Llama-3-8B down_proj FP8 W8A8 N=4096 K=14336 M=64", "fp8",
                    lambda: W.fp8_layer(m=64, n=4096, k=14336)))
    entries.append(("Qwen2-7B MLP up INT8 W8A8 N=18944 K=3584 M=32", "int8", lambda: W.int8_layer(m=32)))
    return entries


DECODE_SHAPES = [("Llama-3-8B down_proj", 4096, 14336), ("Llama-3-8B k_proj", 1024, 4096),
                 ("Qwen2-7B q_proj", 3584, 3584), ("Qwen2-7B down_proj", 3584, 18944)]

# The reference's published microbenchmark (RTX PRO 6000 Blackwell, N = K =
# 4096, bf16 x, seed 205; the reference's
# bench/results/quant-gemm-rtxpro6000-2026-07-27.json): median ms of
# module(x) per scheme and M.
REFERENCE_MICROBENCH_MS = {("fp8", 1): 0.11891, ("fp8", 128): 0.11754, ("int8", 1): 0.10899,
                           ("int8", 128): 0.11770, ("awq", 1): 0.08890, ("awq", 128): 0.29862,
                           ("gptq", 1): 0.10749, ("gptq", 128): 0.26109}


def _eager_median_ms(fn, warmup: int = 50, repeats: int = 200) -> float:
    """The reference microbenchmark's timing (quant_gemm_bench.py:70-97):
    events around each eager call, one synchronize after all samples, median."""

    import statistics

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    for start, end in zip(starts, ends):
        start.record()
        fn()
        end.record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in zip(starts, ends))


def reference_microbench_rows() -> list[dict]:
    """Context rows at the reference microbenchmark's own setup (N = K = 4096,
    M in {1, 128}, bf16 x, seed 205, FP8 / INT8 / AWQ / GPTQ): the module call
    timed the reference's way (eager events, median of 200 after 50 warm-ups,
    the weights not rotated, so they may sit in the MALL as on the reference's
    run) and this bench's way (graph samples, weights rotated past the MALL),
    next to the reference's published time on its own hardware (context, not
    a parity target), and the output against the oracle."""

    import torch

    from kairyu_amd import workloads as W
    from oracle import linear as olinear

    rows = []
    for scheme in ("fp8", "int8", "awq", "gptq"):
        for m in (1, 128):
            wl = W.reference_microbench_layer(scheme, m)
            eager = _eager_median_ms(lambda wl=wl: wl.module(wl.x))
            graph = measure(wl, 20, 5)
            out = wl.module(wl.x)
            torch.cuda.synchronize()
            mod = wl.module
            x32 = _np(wl.x)
            if scheme in ("awq", "gptq"):
                args = (x32, mod.qweight.cpu().numpy(), mod.qzeros.cpu().numpy(), _np(mod.scales))
                expected = (olinear.awq_forward(*args, mod.group_size, "bfloat16") if scheme == "awq"
                            else olinear.gptq_forward(*args, mod.g_idx.cpu().numpy(), "bfloat16"))
            elif scheme == "fp8":
                expected, *_ = olinear.fp8_forward(x32, _bits_np(mod.weight), _np(mod.weight_scale))
            else:
                expected, *_ = olinear.int8_forward(x32, mod.weight.cpu().numpy(), _np(mod.weight_scale), None)
            err = olinear.error_metrics(_np(out), expected)
            ref_ms = REFERENCE_MICROBENCH_MS[(scheme, m)]
            rows.append({
                "scheme": scheme, "shape": {"m": m, "n": 4096, "k": 4096}, "x_dtype": "bfloat16", "seed": 205,
                "eager_median_us": round(eager * 1e3, 2), "graph_us": round(graph["ms"] * 1e3, 2),
                "reference_rtx_pro_6000_us": round(ref_ms * 1e3, 2),
                "reference_us_over_eager_us": round(ref_ms / eager, 2),
                "vs_oracle": {"rel_rmse": err["rel_rmse"], "normwise_max": err["normwise_max"]},
            })
            print(f"[bench] context {scheme} M={m}: eager {eager * 1e3:.2f} us, graph "
                  f"{graph['ms'] * 1e3:.2f} us (reference on RTX PRO 6000: {ref_ms * 1e3:.2f} us); "
                  f"rel_rmse {err['rel_rmse']:.2e}", file=sys.stderr, flush=True)
            del wl
            torch.cuda.empty_cache()
    return rows


# ---------------------------------------------------------- measured peaks
PEAK_KIND = {"fp16": (0, 16384, 4096), "fp8": (1, 65536, 2048), "int8": (2, 32768, 4096)}


def measure_peaks() -> dict:
    """The box's own ceilings (kq_peak_* in the library): a streaming read of
    a 1 GiB device buffer (the sustained rate, best workgroup count), the same
    kernel over 64 MiB passes rotating through that buffer (a decode GEMM's
    per-launch size, launch ramp included; 1 GiB is four times the MALL), and
    a register-only MFMA loop per matrix instruction (fp16 16x16x32, e4m3
    16x16x128 with unit scales, int8 16x16x64), each timed as a graph of its
    launches (HIP events, median of 7 samples).  Vendor peaks beside them."""

    import torch

    from kairyu_amd import _native

    dev = torch.device("cuda", 0)
    sink = torch.zeros(8192 * 256, dtype=torch.int32, device=dev)
    out: dict = {"command": "python bench.py --peaks"}
    big = torch.ones(1 << 30, dtype=torch.uint8, device=dev)

    def read(ptr, nbytes, wg):
        _native.call("kq_peak_stream_read", ptr, nbytes, wg, sink.data_ptr(), _native.stream_handle(dev))

    best = None
    for wg in (1024, 2048, 4096, 8192):
        ms = _graph_ms(lambda i, wg=wg: read(big.data_ptr(), big.numel(), wg), 1, 10)
        rate = big.numel() / (ms * 1e-3) / 1e9
        if best is None or rate > best[0]:
            best = (rate, wg, ms)
    out["hbm_stream_read"] = {"bytes": big.numel(), "workgroups": best[1], "us": round(best[2] * 1e3, 2),
                              "gb_per_s": round(best[0], 1), "frac_of_vendor": round(best[0] / HBM_PEAK_GBS, 4)}
    chunk = 64 << 20
    passes = big.numel() // chunk
    rows = {}
    for wg in (256, 2048):
        ms = _graph_ms(lambda i, wg=wg: read(big.data_ptr() + (i % passes) * chunk, chunk, wg), passes, 200)
        rows[str(wg)] = {"us": round(ms * 1e3, 2), "gb_per_s": round(chunk / (ms * 1e-3) / 1e9, 1)}
    out["hbm_64mib_passes"] = {"bytes": chunk, "rotating_over": big.numel(), "by_workgroups": rows}
    del big
    out["mfma"] = {}
    for name, (kind, flop, iters) in PEAK_KIND.items():
        best = None
        for wg in (512, 1024):
            ms = _graph_ms(lambda i, kind=kind, iters=iters, wg=wg: _native.call(
                "kq_peak_mfma", kind, iters, wg, sink.data_ptr(), _native.stream_handle(dev)), 1, 10)
            tf = wg * 4 * iters * 8 * flop / (ms * 1e-3) / 1e12
            if best is None or tf > best[0]:
                best = (tf, wg, ms)
        out["mfma"][name] = {"tflops": round(best[0], 1), "workgroups": best[1],
                             "us": round(best[2] * 1e3, 2),
                             "frac_of_vendor": round(best[0] / MFMA_PEAK_TFLOPS[name], 4)}
    torch.cuda.synchronize()
    return out


def with_measured_peak(entry: dict | None, peaks: dict | None, dtype: str) -> None:
    """Add the fraction of the box's measured ceiling next to the vendor one."""

    if entry is None or peaks is None:
        return
    if entry.get("unit") == "GB/s":
        measured = peaks["hbm_stream_read"]["gb_per_s"]
    else:
        measured = peaks["mfma"][dtype]["tflops"]
    entry["measured_peak"] = measured
    entry["frac_of_measured_peak"] = round(entry["achieved"] / measured, 4)


def summarize(name: str, dtype: str, workload, result: dict) -> dict:
    frac_hbm = result["gbps"] / HBM_PEAK_GBS
    frac_mfma = result["tflops"] / MFMA_PEAK_TFLOPS[dtype]
    return {
        "name": name,
        "workload": workload.name,
        "bound": workload.bound,
        "ms": round(result["ms"], 5),
        "us": round(result["ms"] * 1e3, 2),
        "gb_per_s": round(result["gbps"], 1),
        "tflops": round(result["tflops"], 2),
        "frac_hbm": round(frac_hbm, 4),
        "frac_mfma": round(frac_mfma, 4),
        "algorithmic_bytes": workload.bytes,
        "flops": workload.flops,
        "weight_copies": result["copies"],
        "timing": result["timing"],
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-sweep", action="store_true")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-headline", action="store_true",
                        help="skip the headline measurement (profiling one sweep row)")
    parser.add_argument("--only", default=None,
                        help="substring filter for sweep entries ('a|b': either)")
    parser.add_argument("--floors", action="store_true",
                        help="only time an empty kernel per step of a HIP graph (the launch floor)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run 256 MiB device-to-device copies (HBM counter calibration)")
    parser.add_argument("--peaks", action="store_true",
                        help="only measure the box's streaming-read and MFMA-loop ceilings")
    parser.add_argument("--no-peaks", action="store_true",
                        help="skip the measured ceilings in a full run")
    parser.add_argument("--no-context", action="store_true",
                        help="skip the reference microbenchmark's context rows")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only in this build)", file=sys.stderr)
        return 2

    import torch

    from kairyu_amd import workloads as W

    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    torch.cuda.set_device(0)
    if args.floors:
        # torch's spin kernel with a zero cycle count: a launch that does no
        # work, 100 per captured graph
        clock_warmup(0.5)
        ms = _graph_ms(lambda i: torch.cuda._sleep(0), 1, 100)
        print(json.dumps({"empty_kernel_per_graph_step_us": round(ms * 1e3, 3)}), flush=True)
        return 0
    if args.copy_calibration:
        # a plain copy of known size: FETCH_SIZE / WRITE_SIZE per dispatch of
        # this kernel calibrate the counters against 268435456 bytes each way
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel(), "copies": 5}), flush=True)
        return 0

    if args.peaks:
        clock_warmup(0.5)
        print(json.dumps({"peaks": measure_peaks()}), flush=True)
        return 0

    clock_warmup()
    peaks = None
    if not args.no_peaks:
        peaks = measure_peaks()
        print(f"[bench] peaks: stream read {peaks['hbm_stream_read']['gb_per_s']} GB/s; MFMA "
              + ", ".join(f"{k} {v['tflops']} TFLOP/s" for k, v in peaks["mfma"].items()),
              file=sys.stderr, flush=True)
    head = kernel = head_summary = None
    if not args.no_headline:
        headline_wl = W.gptq_layer(m=16)
        print(f"[bench] headline {headline_wl.name}", file=sys.stderr, flush=True)
        head = measure(headline_wl, args.steps, args.warmup)
        head_summary = summarize("C2 GPTQ act-order W4A16 N=28672 K=4096 g128 M=16", "fp16",
                                 headline_wl, head)
        kernel = measure_gemm(headline_wl, args.steps, "fp16")
        with_measured_peak(kernel, peaks, "fp16")
        print(f"[bench] headline {head['ms'] * 1e3:.2f} us per op, decode GEMV "
              f"{kernel['us']:.2f} us per launch", file=sys.stderr, flush=True)
        del headline_wl
        torch.cuda.empty_cache()

    sweep = []
    if not args.no_sweep:
        for name, dtype, builder in sweep_entries():
            if args.only and not any(part in name for part in args.only.split("|")):
                continue
            wl = builder()
            print(f"[bench] sweep {name}", file=sys.stderr, flush=True)
            row = summarize(name, dtype, wl, measure(wl, max(20, min(args.steps, 100)),
                                                     min(args.warmup, 10)))
            row["gemm"] = measure_gemm(wl, max(20, min(args.steps, 100)), dtype)
            with_measured_peak(row["gemm"], peaks, dtype)
            print(f"[bench]   op {row['us']} us  {row['gb_per_s']} GB/s  {row['tflops']} TFLOPS"
                  + (f"; gemm {row['gemm']['us']} us {row['gemm']['achieved']} {row['gemm']['unit']}"
                     if row["gemm"] else ""), file=sys.stderr, flush=True)
            vendor = vendor_gemm(wl, max(20, min(args.steps, 100)))
            if vendor is not None:
                row["vendor_gemm"] = vendor
                if "us" in vendor:
                    vendor["vendor_us_over_ours"] = round(vendor["us"] / row["gemm"]["us"], 3)
                    print(f"[bench]   vendor {vendor['us']} us {vendor['achieved']} TFLOP/s "
                          f"({vendor['library']})", file=sys.stderr, flush=True)
            if not args.no_cpu:
                out = wl.module(wl.x)
                torch.cuda.synchronize()
                shape_row = any(name.startswith(label) for label, _, _ in DECODE_SHAPES)
                row["cpu_baseline"], row["parity"] = cpu_row(name, wl, out, target_s=0.5 if shape_row else 2.0)
                print(f"[bench]   cpu {row['cpu_baseline']['value']} {row['cpu_baseline']['unit']}; "
                      f"parity {row['parity']['verdict']}", file=sys.stderr, flush=True)
            sweep.append(row)
            del wl
            torch.cuda.empty_cache()

    context = None
    if not args.no_context and not args.only:
        context = reference_microbench_rows()

    if head is None:
        print(json.dumps({"peaks": peaks, "sweep": sweep, "context": context}), flush=True)
        return 0

    traffic = None
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.is_file():
        traffic = json.loads(traffic_file.read_text()).get(head_summary["workload"])

    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": baseline["metric"],
        "value": round(head["gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded torch.Generator; no checkpoint)",
        "config": {
            "workload": "BASELINE configs[1]: GPTQ act-order W4A16 N=28672 K=4096 group=128, M=16 decode",
            "m": 16, "n": 28672, "k": 4096, "group_size": 128, "act_order": True,
            "x_dtype": "float16", "weight_copies": head["copies"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "w4a16_gemv_kernel (kq_w4a16_tiled_gemm, M=16 decode GEMV)",
            "achieved": kernel["achieved"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": kernel["frac"],
            "traffic": traffic,
            "bytes_per_launch": kernel["bytes_per_launch"],
            "us_per_launch": kernel["us"],
            "timing": kernel["timing"],
            "measured_peak": kernel.get("measured_peak"),
            "frac_of_measured_peak": kernel.get("frac_of_measured_peak"),
        },
        "timing": head["timing"],
        "peaks": peaks,
        "cpu_baseline": cpu,
        "sweep": sweep,
        "context": context,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
