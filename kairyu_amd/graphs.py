"""HIP-graph capture of decode steps over batch buckets.

The reference captures its decode step once per batch bucket and replays it
(``kairyu/engine/core/graph_buckets.py:5-28`` for the bucket policy,
``kairyu/engine/core/cuda_graph_gpu.py:13-91`` for the backend: warm-up on a
side stream, one memory pool shared by every bucket, replay returning the
captured output).  This module keeps that policy and backend contract for the
quantized linears of this package, whose kernels allocate nothing per call
and launch on torch's current stream, so a step built from them captures as
is.  ``BucketedGraphs`` adds what a decode loop needs around it: a static
input per bucket, zero padding for the rows a batch does not fill, and eager
execution for batches beyond the largest bucket.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

_SMALL = (1, 2, 4, 8, 16, 24, 32)
_STEP = 8


def decode_buckets(max_batch: int) -> tuple[int, ...]:
    """Capture sizes: 1, 2, 4, 8, 16, 24, 32, then steps of 8, then
    ``max_batch`` itself (graph_buckets.py:9-20)."""

    if max_batch < 1:
        raise ValueError("max_batch must be >= 1")
    sizes = [b for b in _SMALL if b <= max_batch]
    nxt = _SMALL[-1] + _STEP
    while nxt <= max_batch:
        sizes.append(nxt)
        nxt += _STEP
    if sizes[-1] != max_batch:
        sizes.append(max_batch)
    return tuple(sizes)


def bucket_for(batch_size: int, buckets: tuple[int, ...]) -> int | None:
    """Smallest bucket holding ``batch_size`` rows; ``None``: run eagerly
    (graph_buckets.py:23-28)."""

    for b in buckets:
        if b >= batch_size:
            return b
    return None


class HipGraphBackend:
    """Capture / replay with the reference backend's contract
    (cuda_graph_gpu.py:13-91): ``warmup_iters`` forwards on a side stream,
    then one forward inside ``torch.cuda.graph`` using a pool shared by all
    captures; ``replay()`` re-runs the recorded kernels on the captured
    buffers and returns the captured output."""

    def __init__(self, warmup_iters: int = 3) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("HipGraphBackend requires a ROCm device")
        if warmup_iters < 0:
            raise ValueError(f"warmup_iters must be >= 0, got {warmup_iters}")
        self._warmup_iters = warmup_iters
        self._pool = torch.cuda.graph_pool_handle()
        self.captures = 0
        self.replays = 0

    @property
    def capture_model_forward_count(self) -> int:
        return self._warmup_iters + 1

    def invalidate(self) -> None:
        """Start a new pool: outputs of earlier graphs may still be held."""

        self._pool = torch.cuda.graph_pool_handle()

    def capture(self, fn: Callable[[torch.Tensor], torch.Tensor], static_input: torch.Tensor):
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(self._warmup_iters):
                fn(static_input)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._pool):
            static_out = fn(static_input)
        self.captures += 1
        return _Replayable(self, graph, static_out)


class _Replayable:
    def __init__(self, backend: HipGraphBackend, graph: torch.cuda.CUDAGraph,
                 out: torch.Tensor) -> None:
        self._backend = backend
        self._graph: torch.cuda.CUDAGraph | None = graph
        self._out: torch.Tensor | None = out

    def replay(self) -> torch.Tensor:
        if self._graph is None or self._out is None:
            raise RuntimeError("replay of a closed graph")
        self._backend.replays += 1
        self._graph.replay()
        return self._out

    def close(self) -> None:
        self._graph = None
        self._out = None


class BucketedGraphs:
    """A row-wise step ``fn(x[B, K]) -> y[B, N]`` captured once per bucket.

    ``run(x)`` copies ``x`` into the smallest bucket's static input (rows past
    ``x`` zero), replays that bucket's graph and returns the first rows of its
    output (a view of the captured buffer, valid until the next replay of the
    bucket); batches above the largest bucket run ``fn`` eagerly.  ``fn`` must
    treat rows independently, as the quantized linears do (per-token
    activation scales), so padding rows never change the real rows.
    """

    def __init__(self, fn: Callable[[torch.Tensor], torch.Tensor], in_features: int,
                 max_batch: int, *, dtype: torch.dtype, device: torch.device | str,
                 backend: HipGraphBackend | None = None) -> None:
        self._fn = fn
        self._k = in_features
        self.buckets = decode_buckets(max_batch)
        self._backend = backend or HipGraphBackend()
        self._inputs: dict[int, torch.Tensor] = {}
        self._graphs: dict[int, _Replayable] = {}
        self._dtype = dtype
        self._device = torch.device(device)

    def capture_all(self) -> None:
        """Capture every bucket (smallest first); on a failure the buckets
        captured so far are released before the error propagates."""

        try:
            for b in self.buckets:
                if b in self._graphs:
                    continue
                x = torch.zeros((b, self._k), dtype=self._dtype, device=self._device)
                self._inputs[b] = x
                self._graphs[b] = self._backend.capture(self._fn, x)
        except Exception:
            self.close()
            raise

    def run(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.shape[0]
        b = bucket_for(rows, self.buckets)
        if b is None or b not in self._graphs:
            return self._fn(x)
        static = self._inputs[b]
        static[:rows].copy_(x)
        if rows < b:
            static[rows:].zero_()
        return self._graphs[b].replay()[:rows]

    def invalidate(self) -> None:
        """Drop every graph (weights were swapped); the next capture_all re-records."""

        self.close()
        self._backend.invalidate()

    def close(self) -> None:
        for g in self._graphs.values():
            g.close()
        self._graphs.clear()
        self._inputs.clear()
