"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (``value``): GPTQ act-order W4A16 (N=28672,
K=4096, group 128) at decode size M=16, as whole-op HBM throughput in GB/s of
algorithmic bytes.  One step = one forward of the quantized linear on one
batch; weights rotate over enough distinct HBM copies (> 256 MB MALL) that no
step is served from the Infinity Cache.  Steps are captured in a HIP graph and
timed with HIP events on the stream they run on.

``roofline`` describes the dominant kernel alone: the decode GEMV's
algorithmic bytes per launch over its per-launch time, timed live with HIP
events on its own captured launches (x gathered once up front).

``sweep`` reports every BASELINE configuration (C1-C4 over their M values, C5
when built) with GB/s or TFLOPS and roofline fractions.  ``cpu_baseline``
times the repo's CPU oracle (a numpy port of the reference's dequantize-then-
matmul path) on a bounded sample of the headline workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
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


def _timed_replays(graph, steps: int, repeats: int = 3, settle_s: float = 0.3) -> float:
    """Median over `repeats` timed replays of ms per captured step (HIP events
    on the replaying stream).  Untimed replays first, for at least `settle_s`
    seconds: the GPU idles while the host builds a workload and its graph, and
    its clocks need that long under load to return to their steady state."""

    import torch

    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < settle_s:
        graph.replay()
        torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    return sorted(times)[len(times) // 2]


def measure_headline_kernel(workload, steps: int) -> dict:
    """Live per-launch time of the headline's dominant kernel (the W4A16
    decode GEMV) alone: the act-order gather is done once up front and each
    captured step is one kq_w4a16_tiled_gemm launch on the gathered fp16 x,
    rotating over the same weight copies as the whole-op measurement."""

    import torch

    from kairyu_amd import _native, workloads
    from kairyu_amd.kernels import quant_gemm_hip as hip

    module = workload.module
    copies = max(1, math.ceil(1.25 * MALL_BYTES / max(1, _weight_bytes(module))))
    copies = min(copies, 64)
    mods = workloads.replicas(workload, copies)
    device = workload.x.device
    m, k = workload.x.shape
    n, group = module.out_features, module.group_size
    operands = [hip._gptq_operands(mod, device) for mod in mods]
    mode, _, perm = operands[0]
    x16 = workload.x[:, perm.long()].contiguous() if mode == hip.GIDX_PERMUTED else workload.x
    out = torch.empty((m, n), device=device, dtype=torch.float16)
    ws = _native.workspace(device)

    def launch(i):
        _, tiles, _ = operands[i % copies]
        mod = mods[i % copies]
        _native.call(
            "kq_w4a16_tiled_gemm", x16.data_ptr(), _native.DTYPE_F16, tiles.data_ptr(),
            mod.qzeros.data_ptr(), 1, mod.scales.data_ptr(), None, None, _native.DTYPE_NONE,
            out.data_ptr(), m, n, k, group, ws.data_ptr(), ws.numel(),
            _native.stream_handle(device),
        )

    for i in range(copies):
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
    ms = _timed_replays(graph, steps)
    del graph
    # bytes one launch reads and writes: packed weights, zeros, scales, x16, out
    groups = -(-k // group)
    nbytes = k * n // 2 + groups * (n // 8) * 4 + groups * n * 2 + m * k * 2 + m * n * 2
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9}


def measure(workload, steps: int, warmup: int) -> dict:
    import torch

    from kairyu_amd import workloads

    copies = max(1, math.ceil(1.25 * MALL_BYTES / max(1, _weight_bytes(workload.module))))
    copies = min(copies, 64)
    mods = workloads.replicas(workload, copies)
    x = workload.x
    for i in range(max(warmup, copies)):
        mods[i % copies](x)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(copies):
            mods[i](x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            mods[i % copies](x)
    ms = _timed_replays(graph, steps)
    del graph
    gbps = workload.bytes / (ms * 1e-3) / 1e9
    tflops = workload.flops / (ms * 1e-3) / 1e12
    return {"ms": ms, "gbps": gbps, "tflops": tflops, "copies": copies}


def sweep_entries(include_moe: bool = True):
    from kairyu_amd import workloads as W

    entries = [("C1 AWQ W4A16 N=K=4096 g128", "fp16", lambda: W.awq_layer(m=16))]
    for m in (1, 4, 16, 64, 512):
        entries.append((f"C2 GPTQ act-order W4A16 N=28672 K=4096 g128 M={m}", "fp16",
                        lambda m=m: W.gptq_layer(m=m)))
    for m in (1, 16, 2048, 8192):
        entries.append((f"C3 FP8 W8A8 N=4096 K=14336 M={m}", "fp8", lambda m=m: W.fp8_layer(m=m)))
    for m in (16, 4096):
        entries.append((f"C4 INT8 W8A8 N=18944 K=3584 M={m}", "int8", lambda m=m: W.int8_layer(m=m)))
    if include_moe:
        try:
            from kairyu_amd import moe  # noqa: F401

            if hasattr(W, "moe_layer"):
                entries.append(("C5 block-FP8 MoE E=128 H=2048 I=768 T=4096 top8", "fp8",
                                lambda: W.moe_layer()))
        except ImportError:
            pass
    return entries


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
    }


def cpu_baseline(target_seconds: float = 12.0) -> dict:
    """Time the oracle's GPTQ act-order forward on a column slice of the
    headline workload (M=16, K=4096, N=7168 of 28672) on this host."""

    import numpy as np
    from threadpoolctl import threadpool_info

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
    olinear.gptq_forward_fast(x, qweight, qzeros, scales, g_idx, "float16")  # warm up
    times = []
    deadline = time.perf_counter() + target_seconds
    while time.perf_counter() < deadline or len(times) < 3:
        t0 = time.perf_counter()
        olinear.gptq_forward_fast(x, qweight, qzeros, scales, g_idx, "float16")
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    med = float(np.median(times))
    blas_threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": int(blas_threads),
        "kind": "port",
        "sample": (f"oracle.linear.gptq_forward_fast (numpy dequantize -> fp16 weight -> fp32 BLAS "
                   f"matmul) on M=16 K=4096 N=7168 (1/4 of C2's columns), median of {len(times)} "
                   f"runs = {med * 1e3:.1f} ms; host os.cpu_count()={os.cpu_count()}"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-sweep", action="store_true")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--only", default=None, help="substring filter for sweep entries")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run 256 MiB device-to-device copies (HBM counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only in this build)", file=sys.stderr)
        return 2

    import torch

    from kairyu_amd import workloads as W

    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    torch.cuda.set_device(0)
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

    clock_warmup()
    headline_wl = W.gptq_layer(m=16)
    print(f"[bench] headline {headline_wl.name}", file=sys.stderr, flush=True)
    head = measure(headline_wl, args.steps, args.warmup)
    head_summary = summarize("C2 GPTQ act-order W4A16 N=28672 K=4096 g128 M=16", "fp16",
                             headline_wl, head)
    kernel = measure_headline_kernel(headline_wl, args.steps)
    print(f"[bench] headline {head['ms'] * 1e3:.2f} us per op, decode GEMV "
          f"{kernel['ms'] * 1e3:.2f} us per launch", file=sys.stderr, flush=True)
    del headline_wl
    torch.cuda.empty_cache()

    sweep = []
    if not args.no_sweep:
        for name, dtype, builder in sweep_entries():
            if args.only and args.only not in name:
                continue
            wl = builder()
            print(f"[bench] sweep {name}", file=sys.stderr, flush=True)
            res = measure(wl, max(20, min(args.steps, 100)), min(args.warmup, 10))
            sweep.append(summarize(name, dtype, wl, res))
            print(f"[bench]   {sweep[-1]['us']} us  {sweep[-1]['gb_per_s']} GB/s  "
                  f"{sweep[-1]['tflops']} TFLOPS", file=sys.stderr, flush=True)
            del wl
            torch.cuda.empty_cache()

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
            "achieved": round(kernel["gbps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel["gbps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": kernel["bytes"],
            "us_per_launch": round(kernel["ms"] * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
