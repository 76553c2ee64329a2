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

import glob
import math
import os
import re
import statistics
import threading
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

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


# --------------------------------------------------------------------------
# Clock, power and temperature of the GPU (the reference samples the SM clock
# around each timing with nvidia-smi, bench/harness.py:49-57, :69-89).  Here
# the amdgpu driver's sysfs files of torch device 0 are read directly -- no
# helper process -- by a thread that polls them through the timed window, so
# a clock drop during the run is seen, not only the idle clock before/after.
# --------------------------------------------------------------------------
class GpuTelemetry:
    """Readings of one GPU's amdgpu sysfs node (None where a file is
    missing or unreadable): shader and memory clock in MHz (the active DPM
    level, or the hwmon frequency), board power in W, edge/hotspot
    temperature in C."""

    def __init__(self, device: int = 0):
        self.path = self._find(device)
        hw = glob.glob(os.path.join(self.path, "hwmon", "hwmon*")) if self.path else []
        self.hwmon = hw[0] if hw else None

    @staticmethod
    def _find(device: int) -> Optional[str]:
        try:
            p = torch.cuda.get_device_properties(device)
            addr = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
        except Exception:  # noqa: BLE001 -- no GPU / older torch: no telemetry
            return None
        path = os.path.join("/sys/bus/pci/devices", addr)
        return path if os.path.isdir(path) else None

    @staticmethod
    def _read(path: Optional[str]) -> Optional[str]:
        if not path:
            return None
        try:
            with open(path) as fh:
                return fh.read()
        except OSError:
            return None

    def _dpm_mhz(self, name: str) -> Optional[float]:
        text = self._read(os.path.join(self.path, name) if self.path else None)
        if not text:
            return None
        for line in text.splitlines():
            if line.rstrip().endswith("*"):
                m = re.search(r"(\d+)\s*[Mm]hz", line)
                if m:
                    return float(m.group(1))
        return None

    def _hwmon(self, name: str, scale: float) -> Optional[float]:
        text = self._read(os.path.join(self.hwmon, name) if self.hwmon else None)
        try:
            return float(text) * scale if text else None
        except ValueError:
            return None

    def sample(self) -> Dict[str, Optional[float]]:
        sclk = self._dpm_mhz("pp_dpm_sclk")
        if sclk is None:
            sclk = self._hwmon("freq1_input", 1e-6)
        power = self._hwmon("power1_average", 1e-6)
        if power is None:
            power = self._hwmon("power1_input", 1e-6)
        return {"sclk_mhz": sclk, "mclk_mhz": self._dpm_mhz("pp_dpm_mclk"), "power_w": power,
                "temp_c": self._hwmon("temp1_input", 1e-3),
                "temp_hotspot_c": self._hwmon("temp2_input", 1e-3)}


_telemetry: Optional[GpuTelemetry] = None


def telemetry() -> GpuTelemetry:
    global _telemetry
    if _telemetry is None:
        _telemetry = GpuTelemetry(0)
    return _telemetry


class ClockMonitor:
    """Samples :class:`GpuTelemetry` every ``period_s`` from a thread between
    ``start()`` and ``stop()``; ``summary()`` gives the first and last shader
    clock, its min / mean / max over the window, mean power and peak
    temperature.  ``throttled`` follows the reference's test -- the clock
    moving by more than 5% -- applied to the whole window."""

    def __init__(self, period_s: float = 0.01):
        self.period = period_s
        self.samples: List[Dict[str, Optional[float]]] = []
        self._stop = threading.Event()
        self._thread: Optional[threading.Thread] = None

    def start(self) -> "ClockMonitor":
        tel = telemetry()
        self.samples = []

        # The thread takes the first sample too: a sysfs read on the caller's
        # thread would hold back the first timed window while the GPU idles.
        def run():
            self.samples.append(tel.sample())
            while not self._stop.wait(self.period):
                self.samples.append(tel.sample())

        self._thread = threading.Thread(target=run, daemon=True)
        self._thread.start()
        return self

    def stop(self) -> Dict[str, object]:
        self._stop.set()
        if self._thread is not None:
            self._thread.join()
        self.samples.append(telemetry().sample())
        return self.summary()

    def summary(self) -> Dict[str, object]:
        def col(key):
            return [s[key] for s in self.samples if s.get(key) is not None]

        sclk, power, temp = col("sclk_mhz"), col("power_w"), col("temp_hotspot_c") or col("temp_c")
        out: Dict[str, object] = {"telemetry_samples": len(self.samples)}
        if sclk:
            out.update(clock_before_mhz=sclk[0], clock_after_mhz=sclk[-1], clock_min_mhz=min(sclk),
                       clock_mean_mhz=round(statistics.mean(sclk), 1), clock_max_mhz=max(sclk),
                       throttled=(max(sclk) - min(sclk)) > 0.05 * max(sclk))
        if col("mclk_mhz"):
            out["mclk_mhz"] = statistics.median(col("mclk_mhz"))
        if power:
            out["power_mean_w"] = round(statistics.mean(power), 1)
        if temp:
            out["temp_max_c"] = max(temp)
        return out


@dataclass(frozen=True)
class Timing:
    """One measurement: the per-call time of each timed window, in ms.

    A window spans ``reps`` calls between two events; ``windows_ms`` holds
    each window's elapsed time divided by ``reps``.  Quantiles interpolate
    linearly between the sorted windows (numpy's default definition)."""

    windows_ms: Tuple[float, ...]
    reps: int
    clocks: Dict[str, object] = field(default_factory=dict)

    @property
    def trials(self) -> int:
        return len(self.windows_ms)

    def quantile_ms(self, q: float) -> float:
        xs = sorted(self.windows_ms)
        if not xs:
            return float("nan")
        pos = q * (len(xs) - 1)
        lo = int(math.floor(pos))
        hi = min(lo + 1, len(xs) - 1)
        return xs[lo] + (pos - lo) * (xs[hi] - xs[lo])

    @property
    def median_ms(self) -> float:
        return self.quantile_ms(0.5)

    @property
    def p05_ms(self) -> float:
        return self.quantile_ms(0.05)

    @property
    def p95_ms(self) -> float:
        return self.quantile_ms(0.95)

    @property
    def throttled(self) -> bool:
        return bool(self.clocks.get("throttled", False))


def _new_event() -> "torch.cuda.Event":
    return torch.cuda.Event(enable_timing=True)


def _time_windows(issue: Callable[[], None], trials: int, per_window: int):
    """``trials`` timed windows of ``issue()`` (``per_window`` calls each)
    between two events on the current stream.  The device is idle when each
    window opens (a synchronisation first), as for a host loop that waits
    for each result -- the reference's protocol (bench/harness.py:103-186).
    Returns (per-call ms of each window, clock summary)."""
    mon = ClockMonitor().start()
    out = []
    for _ in range(trials):
        first, last = _new_event(), _new_event()
        torch.cuda.synchronize()
        first.record()
        issue()
        last.record()
        last.synchronize()
        out.append(first.elapsed_time(last) / per_window)
    return tuple(out), mon.stop()


def keep_busy(issue: Callable[[], None], seconds: float) -> None:
    """Issues ``issue()`` back to back for about ``seconds`` and returns while
    the last call is still running, so what is queued next starts at the
    loaded clock.

    After an idle of a few milliseconds MI355X runs its first millisecond or
    so of full-HBM work at ~2.25 GHz, drops to ~1.6 GHz and climbs back over
    the next ~25 ms (busy-cycle counts per dispatch stay constant while the
    duration moves with the clock).  A timing that opens after such an idle
    measures that dip, so the host waits on an event recorded before the last
    call rather than sleeping for an estimate of the queue's length: a sleep
    that outlasts the queue leaves the GPU idle and starts the dip again."""
    start, end = _new_event(), _new_event()
    start.record()
    issue()
    end.record()
    end.synchronize()
    per = max(start.elapsed_time(end) / 1e3, 1e-6)
    for _ in range(max(1, math.ceil(seconds / per)) - 1):
        issue()
    before_last = _new_event()
    before_last.record()
    issue()
    before_last.synchronize()


def bench(fn: Callable[[int], object], *, reps: int = 32, trials: int = 20,
          warmup: int = 5, warm_s: float = 0.05) -> Timing:
    """Eager timing of ``fn(i)``: windows of ``reps`` calls issued back to
    back, after ``warmup`` calls and ``warm_s`` seconds of untimed windows
    (:func:`keep_busy`).  The call index keeps counting across windows, so a
    rotation of weight copies advances through all of them."""
    for i in range(warmup):
        fn(i)
    index = [0]

    def window():
        for _ in range(reps):
            fn(index[0])
            index[0] += 1

    keep_busy(window, warm_s)
    windows, clocks = _time_windows(window, trials, reps)
    return Timing(windows, reps, clocks)


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

    def warm(self, seconds: float) -> None:
        """Untimed replays for about ``seconds``; returns while the last one
        is still running (:func:`keep_busy`)."""
        keep_busy(self.graph.replay, seconds)

    def time(self, trials: int = 20, warm_s: float = 0.05) -> Timing:
        """``trials`` windows of one replay each, after :meth:`warm`."""
        self.warm(warm_s)
        windows, clocks = _time_windows(self.graph.replay, trials, self.reps)
        return Timing(windows, self.reps, clocks)

    def time_window(self, min_ms: float = 20.0, warm_s: float = 0.25):
        """One timed window of whole replays lasting at least ``min_ms``.

        The replay count comes from an untimed replay's duration, so the
        window's length does not depend on how many calls the graph holds.
        Returns (ms per call, replays, clock summary); ms per call is the
        window over replays x calls per replay."""
        first, last = _new_event(), _new_event()
        first.record()
        self.graph.replay()
        last.record()
        last.synchronize()
        per_replay = max(first.elapsed_time(last), 1e-4)
        replays = max(1, math.ceil(min_ms / per_replay))
        self.warm(warm_s)
        mon = ClockMonitor().start()
        first.record()
        for _ in range(replays):
            self.graph.replay()
        last.record()
        last.synchronize()
        clocks = mon.stop()
        return first.elapsed_time(last) / (replays * self.reps), replays, clocks


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
    for r in runners:
        r.warm(0.025)
    # Alternate the two graphs window by window: the windows come out a, b,
    # a, b, ... and are split back by position.
    turn = [0]

    def one():
        runners[turn[0] % 2].graph.replay()
        turn[0] += 1

    windows, clocks = _time_windows(one, 2 * trials, reps)
    return tuple(Timing(windows[k::2], reps, clocks) for k in (0, 1))


def spin_up(seconds: float = 0.3) -> None:
    """Keep the GPU busy with device copies for about ``seconds`` so the
    shader clock is at its loaded level before a sweep's first timing."""
    src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    dst.copy_(src)
    end.record()
    end.synchronize()
    per = max(start.elapsed_time(end) / 1e3, 1e-6)
    for _ in range(max(1, math.ceil(seconds / per))):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


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


_probe = None


def _read_probe_fn():
    global _probe
    if _probe is None:
        import ctypes  # noqa: PLC0415

        from . import _native  # noqa: PLC0415

        _native.binding()  # fail loudly when the library is not built
        lib = ctypes.CDLL(_native.LIBRARY_PATH)
        fn = lib.nibble_read_probe
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_void_p,
                       ctypes.c_void_p]
        _probe = fn
    return _probe


def measured_read_gbps(size_bytes: int = 2 << 30, workgroups=(2048, 4096, 8192)) -> Dict[str, float]:
    """Achievable HBM read bandwidth: the library's streaming-read probe over
    ``size_bytes`` (>= 2 GiB, eight times the Infinity Cache), best over a few
    workgroup counts.  Returns ``{"read_gbps": ..., "read_workgroups": ...}``."""
    fn = _read_probe_fn()
    src = torch.ones(size_bytes // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(max(workgroups), dtype=torch.int32, device="cuda")
    best = None
    for wgs in workgroups:
        def run(_):
            rc = fn(src.data_ptr(), size_bytes, wgs, sink.data_ptr(),
                    torch.cuda.current_stream().cuda_stream)
            if rc:
                raise RuntimeError(f"read probe failed ({rc})")
        t = bench(run, reps=4, trials=8, warmup=2)
        gbps = size_bytes / (t.median_ms * 1e-3) / 1e9
        if best is None or gbps > best[0]:
            best = (gbps, wgs)
    del src, sink
    torch.cuda.empty_cache()
    return {"read_gbps": round(best[0], 1), "read_workgroups": best[1]}


class Ring:
    """A fixed tuple of objects indexed modulo its length: ``ring[i]`` for any
    call index ``i``.  Timed loops index rings of weight copies this way so
    that consecutive calls read different copies."""

    def __init__(self, items):
        self.items = tuple(items)
        if not self.items:
            raise ValueError("a ring needs at least one item")

    def __len__(self) -> int:
        return len(self.items)

    def __getitem__(self, i: int):
        return self.items[i % len(self.items)]

    def map(self, fn: Callable[[object], object]) -> "Ring":
        return Ring(fn(x) for x in self.items)


def copies_for(nbytes: int, min_total_bytes: int = ROTATION_BYTES, cap: int = 512) -> int:
    """How many copies of an ``nbytes`` object together span
    ``min_total_bytes`` (at least one, at most ``cap``)."""
    if nbytes <= 0:
        return 1
    return max(1, min(cap, math.ceil(min_total_bytes / nbytes)))


def tensor_ring(proto: torch.Tensor, min_total_bytes: int = ROTATION_BYTES,
                cap: int = 512) -> Ring:
    """``proto`` and clones of it, enough to span ``min_total_bytes``."""
    n = copies_for(proto.numel() * proto.element_size(), min_total_bytes, cap)
    return Ring([proto, *(proto.clone() for _ in range(n - 1))])


def weight_ring(qw, min_total_bytes: int = ROTATION_BYTES, cap: int = 512) -> Ring:
    """Copies of a packed weight (``QuantizedWeight``: its int32 words and its
    scales cloned together) spanning ``min_total_bytes``: each call of a
    timed loop then streams its weights from HBM, not from the 256 MiB
    Infinity Cache."""
    n = copies_for(qw.weight_bytes, min_total_bytes, cap)
    same = type(qw)
    return Ring([qw, *(same(qw.qweight.clone(), qw.scales.clone(), qw.group_size, qw.K, qw.N)
                       for _ in range(n - 1))])


def ring_bytes(ring: Ring) -> int:
    """Total bytes held by a ring of tensors or packed weights."""
    total = 0
    for x in ring.items:
        total += x.weight_bytes if hasattr(x, "weight_bytes") else x.numel() * x.element_size()
    return total


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
    """A GitHub table of ``rows`` (dicts; missing keys left blank), with every
    column padded to its widest cell so the text lines up as well."""
    grid = [list(map(str, columns))] + [["" if r.get(c) is None else str(r.get(c))
                                         for c in columns] for r in rows]
    width = [max(len(line[j]) for line in grid) for j in range(len(columns))]
    text = ["| " + " | ".join(cell.ljust(w) for cell, w in zip(line, width)) + " |"
            for line in grid]
    text.insert(1, "| " + " | ".join("-" * w for w in width) + " |")
    return "\n".join(text)
