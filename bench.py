#!/usr/bin/env python3
"""Headline benchmark: the M=1 W4A16 decode GEMV at K=4096, N=14336, g=128.

BASELINE.json's metric is "M=1 W4A16 GEMV us & % HBM peak (4096x14336);
8B-shape decode tok/s", quoted on configs[1]'s gate/up shape; the second half
(configs[4], the Llama-3-8B-shaped decode step) is reported under
``decode_8b`` by :mod:`nibblegemm_amd.decode_step`, and config 4's M=2048
prefill GEMM points under ``prefill_2048`` (each checked against an fp32
reference before it is timed).  A *step* is
one ``nibblegemm_amd.gemv`` call (M=1) over one batch of synthetic inputs
(nibbles U{0..15}, scales fp16 U(0.002, 0.02), activations fp16 N(0,1)).

* Inputs are resident in HBM before timing.  Each step reads a different copy
  of the packed weights and scales from a rotation spanning >= 1 GiB, so no
  step is served from the 256 MiB Infinity Cache or the L2s.
* ``--warmup W`` eager steps run untimed, then the timed steps are captured
  into one HIP graph (capture executes nothing) of C = max(K,
  ``--min-graph-calls``) calls (1000: each graph launch adds ~3.6 us of its
  own between replays, 3% of a 20-call replay), replayed untimed for ~0.25 s
  so the timed window starts at the loaded shader clock, and then replayed
  R times back to back between two events on the replay stream, bracketed by
  ``torch.cuda.synchronize()``.  R is the smallest count whose window lasts
  at least ``--min-window-ms`` (30 ms), whatever K is, so the figure does not
  depend on K and the sysfs clock / power sampler (10 ms period) sees the
  window: ``ms_per_step`` = window / (R * C), ``timed_replays`` = R and
  ``calls_per_replay`` = C.
  ``clock`` holds the shader clock at the window's start and end, min /
  mean / max over it, and the reference's ``throttled`` test (the clock
  moving by more than 5%).
* ``value`` = algorithmic bytes per step (K*N/2 + (K/128)*N*2 + 2K + 2N) /
  ms_per_step, in GB/s.  ``roofline`` prices the same figure against MI355X's
  8 TB/s; ``cpu_baseline`` times the CPU oracle (dequantize + fp32 matmul,
  the reference's CPU path) on this host on a bounded sample, and its
  ``per_shape`` table the same path at every other shape the line reports
  (decode sweep, small batches, prefill, dequant) on all of the job's cores.
* ``small_batch`` (configs[2]: M = 2..32 through ``matmul`` at the headline
  shape, and M = 16, 24, 32 at 14336 x 4096) and ``dequant`` (the standalone
  kernel at the headline shape, bit-exact first) are graph-timed over the
  same kind of rotation.

Prints ONE JSON line.  Only ``--gpus 1`` is supported (one GPU per box).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "M=1 W4A16 GEMV µs & % HBM peak (4096x14336); 8B-shape decode tok/s"
K, N, M, G = 4096, 14336, 1, 128


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


#: Shapes whose reference CPU path the line reports beside the GPU figures:
#: (M, K, N).  The decode sweep (configs[0..1]), the small batches
#: and the prefill points.
CPU_SHAPES = ([(1, k, n) for k, n in ((4096, 14336), (14336, 4096), (8192, 8192), (4096, 4096),
                                      (4096, 1024), (4096, 6144))]
              + [(m, 4096, 14336) for m in (2, 4, 8, 16, 17, 24, 32)]
              + [(m, 14336, 4096) for m in (16, 24, 32)]
              + [(m, k, n) for m in (128, 512, 2048) for k, n in ((4096, 14336), (14336, 4096))])
#: Rows of X the CPU matmul is timed on at most (scaled by M / rows above it).
CPU_MAX_ROWS = 32


def _threads():
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(affinity, omp) if omp > 0 else affinity), affinity, omp


def cpu_per_shape(O, threads: int) -> list:
    """The reference CPU path at every shape of CPU_SHAPES: the oracle's
    dequantize (whole) and fp32 matmul (on at most CPU_MAX_ROWS rows, scaled
    linearly to M), median of 3 after a warm-up, all of the job's cores."""
    rows = []
    for m, k, n in CPU_SHAPES:
        r = O.time_reference_path(m, k, n, G, reps=3, threads=threads, max_rows=CPU_MAX_ROWS)
        nb = k * n // 2 + (k // G) * n * 2 + m * k * 2 + m * n * 2
        rows.append({"M": m, "K": k, "N": n, "ms": round(r["total_s"] * 1e3, 2),
                     "dequant_ms": round(r["dequant_s"] * 1e3, 2),
                     "matmul_ms": round(r["matmul_s"] * 1e3, 2), "rows_timed": r["rows_timed"],
                     "gbps": round(nb / r["total_s"] / 1e9, 3),
                     "tflops": round(2 * m * k * n / r["total_s"] / 1e12, 4)})
    return rows


def cpu_baseline(target_s: float, per_shape: bool = True) -> dict:
    """The reference's CPU path (dequantize + fp32 matmul), via the CPU oracle,
    on this host's cores: as many threads as the job's CPU share allows (the
    affinity mask, capped by OMP_NUM_THREADS where the box sets it)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # noqa: PLC0415  (cpu_baseline leg only)

    threads, affinity, omp = _threads()
    one = O.time_reference_path(M, K, N, G, reps=1, threads=threads)
    reps = int(max(5, min(60, target_s / max(one["total_s"], 1e-3))))
    r = O.time_reference_path(M, K, N, G, reps=reps, threads=threads)
    nbytes = K * N // 2 + (K // G) * N * 2 + M * K * 2 + M * N * 2
    return {
        "value": round(nbytes / r["total_s"] / 1e9, 3),
        "unit": "GB/s",
        "cores": r["threads"],
        "kind": "port",
        "sample": (f"oracle dequantize + fp32 matmul (the reference CPU path), M=1 K={K} N={N} "
                   f"g={G}, median of {reps} reps after 1 warm-up; dequant "
                   f"{r['dequant_s'] * 1e3:.1f} ms + matmul {r['matmul_s'] * 1e3:.1f} ms "
                   f"= {r['total_s'] * 1e3:.1f} ms per step"),
        "ms_per_step": round(r["total_s"] * 1e3, 3),
        "dequant_ms": round(r["dequant_s"] * 1e3, 3),
        "matmul_ms": round(r["matmul_s"] * 1e3, 3),
        "threads_used": r["threads"],
        "host_cpu_count": os.cpu_count(),
        "affinity_cores": affinity,
        "omp_num_threads": omp or None,
        "cpu_model": _cpu_model(),
        "per_shape": cpu_per_shape(O, threads) if per_shape else None,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--min-window-ms", type=float, default=30.0,
                    help="shortest timed window; the graph is replayed until it is reached")
    ap.add_argument("--min-graph-calls", type=int, default=1000,
                    help="fewest calls captured in the timed graph (at least --steps)")
    ap.add_argument("--no-cpu-shapes", action="store_true",
                    help="time the CPU path at the headline shape only")
    ap.add_argument("--skip-extras", action="store_true",
                    help="skip the copy-bandwidth, hipBLASLt and eager side measurements")
    ap.add_argument("--skip-decode-step", action="store_true",
                    help="skip the Llama-3-8B-shaped decode step")
    ap.add_argument("--skip-prefill", action="store_true",
                    help="skip the M=2048 prefill GEMM points")
    ap.add_argument("--skip-small-batch", action="store_true",
                    help="skip the small-batch matmul points and the standalone dequant")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the W4A16 path has no multi-GPU leg in this build.", file=sys.stderr)
        return 2
    steps, warmup = max(1, args.steps), max(0, args.warmup)

    import torch  # noqa: PLC0415

    import nibblegemm_amd as ng  # noqa: PLC0415
    from nibblegemm_amd import harness as H  # noqa: PLC0415

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    ng.extension()  # fail loudly if the native library is missing
    dev = torch.device("cuda", 0)
    log(H.device_summary())

    # ---- synthetic inputs (host-generated, seeded), resident in HBM ----------
    gen = torch.Generator().manual_seed(0)
    qu = torch.randint(0, 16, (K, N), generator=gen, dtype=torch.uint8).numpy()
    qweight = torch.from_numpy(ng.pack_nibbles(qu)).to(dev)
    scales = (torch.rand((K // G, N), generator=gen) * 0.018 + 0.002).to(torch.float16).to(dev)
    X = torch.randn((M, K), generator=gen).to(torch.float16).to(dev)
    variants = H.weight_ring(ng.QuantizedWeight(qweight, scales, G, K, N))
    nbytes = H.total_bytes(M, K, N, G, 4)
    log(f"rotation: {len(variants)} copies, {H.ring_bytes(variants) / 2**30:.2f} GiB of packed "
        "weights and scales")

    # ---- warmup (untimed, eager) ---------------------------------------------
    for i in range(warmup):
        ng.gemv(X, variants[i])
    torch.cuda.synchronize()

    # ---- timed steps: one HIP graph of max(K, --min-graph-calls) calls ----------
    calls = max(steps, args.min_graph_calls)
    runner = H.GraphRunner(lambda i: ng.gemv(X, variants[i]), reps=calls, warmup=0)
    runner.graph.replay()  # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    ms_per_step, replays, clocks = runner.time_window(min_ms=args.min_window_ms, warm_s=0.25)
    torch.cuda.synchronize()
    gbps = H.achieved_gbps(nbytes, ms_per_step)
    log(f"gemv M=1 {K}x{N}: {ms_per_step * 1e3:.2f} us/step, {gbps:.0f} GB/s "
        f"({100 * gbps / H.HBM_PEAK_GBPS:.1f}% of 8 TB/s); clock {clocks}")

    extras = {}
    if not args.skip_extras:
        eager = H.bench(lambda i: ng.gemv(X, variants[i]), reps=32, trials=10, warmup=2)
        extras["eager_us_per_call"] = round(eager.median_ms * 1e3, 2)
        copy = H.measured_copy_gbps()
        extras["copy_gbps"] = round(copy, 1)
        extras["pct_of_copy_bw"] = round(100 * gbps / copy, 1)
        read = H.measured_read_gbps()
        extras.update(read)
        extras["pct_of_read_bw"] = round(100 * gbps / read["read_gbps"], 1)
        torch.backends.cuda.matmul.allow_tf32 = False
        w16 = (torch.randn((K, N), generator=gen) * 0.02).to(torch.float16).to(dev)
        rot16 = H.tensor_ring(w16)
        fp16 = H.bench_graph(lambda i: torch.mm(X, rot16[i]), reps=64, trials=10)
        extras["hipblaslt_fp16_us"] = round(fp16.median_ms * 1e3, 2)
        extras["speedup_vs_hipblaslt_fp16"] = round(fp16.median_ms / ms_per_step, 2)
        fp16_bytes = H.total_bytes(M, K, N, G, 16)
        extras["byte_ratio_ceiling"] = round(fp16_bytes / nbytes, 3)
        del rot16, w16
        # The same GEMV on strip-major copies of the rotation (the decode
        # kernel's contiguous-strip layout; same bytes per call).
        sm = variants.map(ng.to_strip_major)
        smt = H.bench_graph(lambda i: ng.matmul(X, sm[i]), reps=64, trials=10)
        extras["strip_major"] = {
            "strip_cols": sm[0].strip_cols, "us": round(smt.median_ms * 1e3, 2),
            "gbps": round(H.achieved_gbps(nbytes, smt.median_ms), 1),
            "pct_hbm_peak": round(100 * H.achieved_gbps(nbytes, smt.median_ms) / H.HBM_PEAK_GBPS, 2),
            "clock_mhz": smt.clocks.get("clock_mean_mhz")}
        del sm
        log(f"copy {copy:.0f} GB/s; 2 GiB read {read['read_gbps']:.0f} GB/s; hipBLASLt fp16 "
            f"{fp16.median_ms * 1e3:.2f} us; eager {eager.median_ms * 1e3:.2f} us/call")

    decode = None
    if not args.skip_decode_step:
        from nibblegemm_amd import decode_step  # noqa: PLC0415

        del variants
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        decode = decode_step.run(32)
        log(f"8B decode step: {decode['projections']['graph_tok_s']} tok/s graph "
            f"({decode['projections']['launches']} launches), fused "
            f"{decode['fused']['graph_tok_s']} tok/s ({decode['fused']['launches']} launches), "
            f"with the SwiGLU epilogue {decode['fused_swiglu']['graph_tok_s']} tok/s; "
            f"full step with norms, attention over {decode['glue']['context']} tokens and "
            f"residual adds {decode['glue']['graph_tok_s']} tok/s ({decode['glue']['launches']} "
            f"launches); strip-major weights: projections "
            f"{decode['projections_strips']['graph_tok_s']}, fused "
            f"{decode['fused_strips']['graph_tok_s']}, SwiGLU "
            f"{decode['fused_swiglu_strips']['graph_tok_s']}, full step "
            f"{decode['glue_strips']['graph_tok_s']} tok/s; as one persistent launch: projections "
            f"{decode['persistent_projections']['graph_tok_s']}, fused "
            f"{decode['persistent']['graph_tok_s']}; on the packed weights unconverted: projections "
            f"{decode['persistent_projections_packed']['graph_tok_s']}, fused "
            f"{decode['persistent_packed']['graph_tok_s']} tok/s; {time.perf_counter() - t0:.1f} s")

    prefill = None
    if not args.skip_prefill:
        from nibblegemm_amd.bench_shapes import prefill_points  # noqa: PLC0415

        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        prefill = [{k: r[k] for k in ("M", "K", "N", "us", "TFLOP/s", "hipblaslt_fp16_us", "vs_fp16",
                                      "max_err_rms")}
                   for KN in ((4096, 14336), (14336, 4096))
                   for r in prefill_points(*KN, [2048], trials=5, versions=(6,))]
        log("prefill M=2048 (gemm v6): " + "; ".join(
            f"{r['K']}x{r['N']} {r['us']} us {r['TFLOP/s']} TFLOP/s ({r['vs_fp16']}x hipBLASLt fp16)"
            for r in prefill) + f"; {time.perf_counter() - t0:.1f} s")

    small = dequant = None
    if not args.skip_small_batch:
        # configs[2]'s small batches through matmul (M <= 8 the decode GEMV,
        # above it the GEMM's plans), and the standalone dequant at the same
        # shape, bit-exact against the host dequantize first.
        from nibblegemm_amd import bench_shapes as BS, quant  # noqa: PLC0415

        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        small = []
        # the headline shape, then the down projection's (K and N swapped)
        for (Ks, Ns), ms in (((K, N), (2, 4, 8, 16, 17, 24, 32)), ((N, K), (16, 24, 32))):
            qws, gen = BS._weights(Ks, Ns, G, seed=Ks + Ns)
            for m in ms:
                Xm = torch.randn((m, Ks), generator=gen).to(torch.float16).cuda()
                err = BS._check(ng.matmul(Xm, qws[0]), Xm, qws[0], f"matmul {m}x{Ks}x{Ns}")
                t = H.bench_graph(lambda i: ng.matmul(Xm, qws[i]), reps=32, trials=10)
                nb = H.total_bytes(m, Ks, Ns, G, 4)
                small.append({"M": m, "K": Ks, "N": Ns, "us": round(t.median_ms * 1e3, 2),
                              "gbps": round(H.achieved_gbps(nb, t.median_ms), 1),
                              "max_err_rms": float(f"{err:.2e}")})
            if (Ks, Ns) == (K, N):
                qws_head = qws
            else:
                del qws
        qws = qws_head
        host = quant.dequantize(qws[0].to("cpu"))
        if not torch.equal(ng.dequant(qws[0]).cpu().view(torch.int16), host.view(torch.int16)):
            raise RuntimeError("dequant differs from the host dequantize")
        t = H.bench_graph(lambda i: ng.dequant(qws[i]), reps=16, trials=10)
        dq_bytes = K * N // 2 + (K // G) * N * 2 + 2 * K * N
        dq_gbps = H.achieved_gbps(dq_bytes, t.median_ms)
        dequant = {"K": K, "N": N, "us": round(t.median_ms * 1e3, 2), "gbps": round(dq_gbps, 1),
                   "pct_hbm_peak": round(100 * dq_gbps / H.HBM_PEAK_GBPS, 2), "bit_exact": True}
        del qws
        log("small batch (matmul): " + "; ".join(f"{r['K']}x{r['N']} M={r['M']} {r['us']} us" for r in small)
            + f"; dequant {dequant['us']} us {dequant['gbps']} GB/s; "
            f"{time.perf_counter() - t0:.1f} s")

    roofline = {
        "bound": "hbm",
        "achieved": round(gbps, 1),
        "peak": H.HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(gbps / H.HBM_PEAK_GBPS, 4),
        "traffic": _committed_traffic(),
    }

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(args.cpu_seconds, per_shape=not args.no_cpu_shapes)
        log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads "
            f"({time.perf_counter() - t0:.1f} s)")

    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "timed_replays": replays,
        "calls_per_replay": calls,
        "timed_window_ms": round(ms_per_step * replays * calls, 3),
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "accumulate": "f32",
        "data": "synthetic",
        "config": {"workload": f"gemv M={M} K={K} N={N} g={G} (BASELINE configs[1] headline shape)",
                   "M": M, "K": K, "N": N, "group_size": G},
        "gemv_us": round(ms_per_step * 1e3, 3),
        "clock": clocks,
        "pct_hbm_peak": round(100 * gbps / H.HBM_PEAK_GBPS, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_8b": decode,
        "prefill_2048": prefill,
        "small_batch": small,
        "dequant": dequant,
        **extras,
    }
    print(json.dumps(line), flush=True)
    return 0


def _committed_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), committed under profiles/."""
    path = os.path.join(ROOT, "profiles", "gemv_m1_4096x14336_traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    sys.exit(main())
