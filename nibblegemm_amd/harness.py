"""Measurement harness for the W4A16 kernels on MI355X.

Restates the reference's bench/harness.py (timing, buffer rotation, copy
bandwidth, traffic model; harness.py:45-259 in arvindcr4/nibblegemm) for the
MI355X memory hierarchy:

* **Cache defeat.** MI355X has 4 MiB of L2 per XCD (8 XCDs, 32 MiB) and a
  256 MiB Infinity Cache (MALL) in front of HBM.  A 4096 x 14336 INT4 weight is
  ~30 MB -- it would be served from the MALL if timed in place.  Rotations are
  sized to at least ``ROTATION_BYTES`` (1 GiB, > 3x L2 + MALL), so every timed
  call streams its weights from HBM.
* **Launch overhead.** A decode GEMV is ~5 us, comparable to a Python-level
  launch.  Kernel time is therefore taken from HIP graph replays of many calls
  (events bracket the replay on the stream the kernels run on); eager timing
  is reported separately.
* **Peak.** Achieved bandwidth is reported against MI355X's 8 TB/s spec and
  against a measured large device copy (>= 2 GiB, read + write counted).
"""
from __future__ import annotations

import statistics
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import torch

#: Total bytes a buffer rotation spans (defeats 32 MiB L2 + 256 MiB MALL).
ROTATION_BYTES = 1 << 30
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E spec
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA spec


def device_summary() -> str:
    p = torch.cuda.get_device_properties(0)
    arch = getattr(p, "gcnArchName", "")
    return (f"{p.name} | {arch} | {p.multi_processor_count} CUs | "
            f"{p.total_memory / 2**30:.0f} GiB HBM")


@dataclass
class Timing:
    median_ms: float
    p05_ms: float
    p95_ms: float
    trials: int
    reps: int
    samples: Sequence[float] = field(default_factory=list, repr=False)

    @property
    def spread_pct(self) -> float:
        return 100.0 * (self.p95_ms - self.p05_ms) / self.median_ms if self.median_ms else 0.0


def _summarise(samples: List[float], trials: int, reps: int) -> Timing:
    samples = sorted(samples)
    return Timing(
        median_ms=statistics.median(samples),
        p05_ms=samples[max(0, int(0.05 * len(samples)) - 1)],
        p95_ms=samples[min(len(samples) - 1, int(0.95 * len(samples)))],
        trials=trials, reps=reps, samples=samples,
    )


def bench(fn: Callable[[int], object], *, reps: int = 32, trials: int = 20,
          warmup: int = 5) -> Timing:
    """Eager: one event pair spans ``reps`` back-to-back calls of ``fn(i)``."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    samples = []
    for _ in range(trials):
        torch.cuda.synchronize()
        start.record()
        for r in range(reps):
            fn(r)
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / reps)
    return _summarise(samples, trials, reps)


class GraphRunner:
    """``reps`` calls of ``fn(i)`` captured into one HIP graph.

    Events are recorded on the replaying (current) stream, the stream the
    captured kernels run on at replay.
    """

    def __init__(self, fn: Callable[[int], object], reps: int, warmup: int = 3):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(warmup):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for r in range(reps):
                fn(r)
        torch.cuda.synchronize()
        self.reps = reps

    def time(self, trials: int = 20) -> Timing:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        self.graph.replay()  # warm
        torch.cuda.synchronize()
        samples = []
        for _ in range(trials):
            start.record()
            self.graph.replay()
            end.record()
            end.synchronize()
            samples.append(start.elapsed_time(end) / self.reps)
        return _summarise(samples, trials, self.reps)


def bench_graph(fn: Callable[[int], object], *, reps: int = 32, trials: int = 20,
                warmup: int = 3) -> Timing:
    return GraphRunner(fn, reps, warmup).time(trials)


def bench_graph_pair(fn_a: Callable[[int], object], fn_b: Callable[[int], object], *,
                     reps: int = 32, trials: int = 20, warmup: int = 3):
    """Two graph-timed candidates with their trials interleaved (a, b, a, b,
    ...), so both see the same clock and thermal state -- a GPU under
    sustained matrix-core load slows down, and timing one candidate after the
    other would charge that to whichever runs second.  Returns (Timing a,
    Timing b)."""
    runners = (GraphRunner(fn_a, reps, warmup), GraphRunner(fn_b, reps, warmup))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    for r in runners:
        r.graph.replay()  # warm
    torch.cuda.synchronize()
    samples = ([], [])
    for _ in range(trials):
        for r, out in zip(runners, samples):
            start.record()
            r.graph.replay()
            end.record()
            end.synchronize()
            out.append(start.elapsed_time(end) / reps)
    return tuple(_summarise(s, trials, reps) for s in samples)


def measured_copy_gbps(size_bytes: int = 2 << 30) -> float:
    """Achievable HBM bandwidth: a large device copy, read + write counted."""
    n = size_bytes // 2
    src = torch.empty(n, dtype=torch.float16, device="cuda")
    src.fill_(1.0)
    dst = torch.empty_like(src)
    t = bench(lambda _: dst.copy_(src), reps=4, trials=10, warmup=2)
    del src, dst
    torch.cuda.empty_cache()
    return (2 * n * 2) / (t.median_ms * 1e-3) / 1e9


class Rotation:
    """Copies of a tensor spanning at least ``min_total_bytes`` in total."""

    def __init__(self, proto: torch.Tensor, min_total_bytes: int = ROTATION_BYTES, cap: int = 512):
        nbytes = proto.numel() * proto.element_size()
        count = max(1, min(cap, -(-min_total_bytes // max(nbytes, 1))))
        self.buffers = [proto] + [proto.clone() for _ in range(count - 1)]
        self.count = len(self.buffers)
        self.total_bytes = self.count * nbytes

    def __getitem__(self, i: int) -> torch.Tensor:
        return self.buffers[i % self.count]


class Cycle:
    def __init__(self, items):
        self.items = list(items)

    def __getitem__(self, i: int):
        return self.items[i % len(self.items)]

    def __len__(self) -> int:
        return len(self.items)


# --------------------------------------------------------------------------
# Traffic model (reference bench/harness.py:243-259)
# --------------------------------------------------------------------------
def weight_bytes(K: int, N: int, group_size: int, bits: int) -> int:
    w = K * N * bits // 8
    s = (K // group_size) * N * 2 if bits < 16 else 0
    return w + s


def total_bytes(M: int, K: int, N: int, group_size: int, bits: int) -> int:
    """Compulsory traffic: weights once, activations in, outputs out."""
    return weight_bytes(K, N, group_size, bits) + M * K * 2 + M * N * 2


def dequant_bytes(K: int, N: int, group_size: int) -> int:
    return K * N // 2 + (K // group_size) * N * 2 + K * N * 2


def achieved_gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


def tflops(M: int, K: int, N: int, ms: float) -> float:
    return (2.0 * M * K * N) / (ms * 1e-3) / 1e12


def markdown_table(rows: Sequence[dict], columns: Sequence[str]) -> str:
    head = "| " + " | ".join(columns) + " |"
    rule = "|" + "|".join("---" for _ in columns) + "|"
    body = ["| " + " | ".join(str(r.get(c, "")) for c in columns) + " |" for r in rows]
    return "\n".join([head, rule, *body])
