"""Shape sweeps of the W4A16 kernels against their baselines on one GPU (the
roles of the reference's bench/bench_decode.py, bench/bench_prefill.py,
bench/launch_overhead.py and bench/autotune.py, at the benchmark shapes).

    python3 -m nibblegemm_amd.bench_shapes decode      # configs 1-3: M <= 8 GEMV
    python3 -m nibblegemm_amd.bench_shapes prefill     # configs 3-4: M = 16 .. 2048
    python3 -m nibblegemm_amd.bench_shapes dequant     # standalone dequant
    python3 -m nibblegemm_amd.bench_shapes crossover   # gemv vs gemm over M (--shape K N)
    python3 -m nibblegemm_amd.bench_shapes strips      # what bounds one decode launch
    python3 -m nibblegemm_amd.bench_shapes launch      # eager vs graph-replayed matmul
    python3 -m nibblegemm_amd.bench_shapes autotune    # gemv splits x block_threads
    python3 -m nibblegemm_amd.bench_shapes attention   # decode-step attention over cache length

Every timing is a HIP-graph replay of many calls; a kernel and its hipBLASLt
baseline are timed with interleaved trials (the same clock state for both).  Each call streams its
weights from HBM: copies of the weights rotate through at least 1 GiB, more
than the 256 MiB Infinity Cache.  Inputs are synthetic, with the benchmark
distributions: nibbles U{0..15}, scales U(0.002, 0.02), activations N(0, 1).
Every measured configuration is first checked against a torch fp32
reference, on the GPU, of the same weights (the bit-exact dequant kernel's
output, multiplied in fp32): max |y - ref| <= 1e-2 * rms(ref), or the sweep
stops.

One JSON object per line on stdout; ``--markdown`` adds a table on stderr.
The reference's CPU path at these shapes is timed by ``bench.py``'s
``cpu_baseline.per_shape`` (the C oracle on all of the job's cores).
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from . import harness as H
from . import ops, quant
from .quant import QuantizedWeight, pack_nibbles

DECODE_SHAPES = [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 8192), (4096, 1024), (4096, 6144)]
PREFILL_SHAPES = [(4096, 14336), (14336, 4096)]
TOL = 1e-2


def _weights(K: int, N: int, G: int, seed: int):
    gen = torch.Generator().manual_seed(seed)
    qu = torch.randint(0, 16, (K, N), generator=gen, dtype=torch.uint8).numpy()
    qweight = torch.from_numpy(pack_nibbles(qu)).cuda()
    scales = (torch.rand((K // G, N), generator=gen) * 0.018 + 0.002).to(torch.float16).cuda()
    return H.weight_ring(QuantizedWeight(qweight, scales, G, K, N)), gen


def _fp16_baseline(qw: QuantizedWeight):
    """fp16 copies of the same (dequantized) weight, rotated through >= 1 GiB."""
    return H.tensor_ring(ops.dequant(qw))


def _check(y: torch.Tensor, X: torch.Tensor, qw: QuantizedWeight, what: str) -> float:
    ref = X.float() @ ops.dequant(qw).float()
    err = float((y.float() - ref).abs().max() / ref.pow(2).mean().sqrt())
    if not err <= TOL:
        raise RuntimeError(f"{what}: max|y - ref| = {err:.3e} * rms(ref) exceeds {TOL}")
    return err


def _emit(rows, row):
    rows.append(row)
    print(json.dumps(row), flush=True)


def _clock(t: "H.Timing") -> dict:
    """The shader clock over a timing's window (mean MHz) and the reference's
    5% throttle flag."""
    c = t.clocks
    return {"clock_mhz": c.get("clock_mean_mhz"), "throttled": c.get("throttled")}


def decode(args, rows):
    copy = H.measured_copy_gbps()
    read = H.measured_read_gbps()["read_gbps"]
    print(json.dumps({"bench": "decode-setup", "copy_gbps": round(copy, 1), "read_gbps": read}),
          flush=True)
    for K, N in DECODE_SHAPES:
        qws, gen = _weights(K, N, args.group_size, seed=K + N)
        w16 = _fp16_baseline(qws[0])
        sms = qws.map(ops.to_strip_major)
        H.spin_up(0.2)  # host-side setup above let the clock drop
        for M in args.M or [1, 2, 4, 8]:
            X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
            err = _check(ops.gemv(X, qws[0]), X, qws[0], f"gemv {M}x{K}x{N}")
            sm_err = _check(ops.matmul(X, sms[0]), X, qws[0], f"strip-major {M}x{K}x{N}")
            t = H.bench_graph(lambda i: ops.gemv(X, qws[i]), reps=64, trials=args.trials)
            ts = H.bench_graph(lambda i: ops.matmul(X, sms[i]), reps=64, trials=args.trials)
            f = H.bench_graph(lambda i: torch.mm(X, w16[i]), reps=64, trials=args.trials)
            d = H.bench_graph(lambda i: torch.mm(X, ops.dequant(qws[i])), reps=8, trials=args.trials)
            nb = H.total_bytes(M, K, N, args.group_size, 4)
            gbps = H.achieved_gbps(nb, t.median_ms)
            row = {"bench": "decode", "M": M, "K": K, "N": N, "impl": "gemv v4",
                   "us": round(t.median_ms * 1e3, 2), "GB/s": round(gbps),
                   "%8TB/s": round(100 * gbps / H.HBM_PEAK_GBPS, 1),
                   "%copy": round(100 * gbps / copy, 1), "%read": round(100 * gbps / read, 1),
                   "hipblaslt_fp16_us": round(f.median_ms * 1e3, 2),
                   "vs_fp16": round(f.median_ms / t.median_ms, 2),
                   "dequant+fp16_us": round(d.median_ms * 1e3, 2),
                   "max_err_rms": float(f"{err:.2e}"), **_clock(t),
                   "strip_cols": sms[0].strip_cols, "strip_major_us": round(ts.median_ms * 1e3, 2),
                   "strip_major_%8TB/s": round(100 * H.achieved_gbps(nb, ts.median_ms)
                                               / H.HBM_PEAK_GBPS, 1),
                   "strip_major_err_rms": float(f"{sm_err:.2e}")}
            _emit(rows, row)
        del qws, w16, sms
        torch.cuda.empty_cache()


def prefill_points(K: int, N: int, Ms, group_size: int = 128, trials: int = 10,
                   versions=(6, 7)):
    """Rows of the prefill sweep at one weight shape (each checked first)."""
    out = []
    qws, gen = _weights(K, N, group_size, seed=K + N)
    w16 = _fp16_baseline(qws[0])
    for M in Ms:
        X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
        reps = 8 if M >= 512 else 32
        for v in versions:
            err = _check(ops.gemm(X, qws[0], version=v), X, qws[0], f"gemm v{v} {M}x{K}x{N}")
            t, f = H.bench_graph_pair(lambda i: ops.gemm(X, qws[i], version=v),
                                      lambda i: torch.mm(X, w16[i]), reps=reps, trials=trials)
            tf = H.tflops(M, K, N, t.median_ms)
            out.append({"bench": "prefill", "M": M, "K": K, "N": N, "impl": f"gemm v{v}",
                        "us": round(t.median_ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                        "%2.5PF": round(100 * tf / H.FP16_MFMA_PEAK_TFLOPS, 1),
                        "hipblaslt_fp16_us": round(f.median_ms * 1e3, 2),
                        "vs_fp16": round(f.median_ms / t.median_ms, 2),
                        "max_err_rms": float(f"{err:.2e}"), **_clock(t)})
    del qws, w16
    torch.cuda.empty_cache()
    return out


def prefill(args, rows):
    for K, N in PREFILL_SHAPES:
        for row in prefill_points(K, N, args.M or [16, 32, 128, 512, 2048], args.group_size,
                                  args.trials):
            _emit(rows, row)


def dequant(args, rows):
    copy = H.measured_copy_gbps()
    print(json.dumps({"bench": "dequant-setup", "copy_gbps": round(copy, 1)}), flush=True)
    for K, N in DECODE_SHAPES:
        qws, _ = _weights(K, N, args.group_size, seed=K + N)
        qw_cpu = qws[0].to("cpu")
        host_w = quant.dequantize(qw_cpu)
        if not torch.equal(ops.dequant(qws[0]).cpu().view(torch.int16), host_w.view(torch.int16)):
            raise RuntimeError(f"dequant {K}x{N}: device result differs from the host dequantize")
        H.spin_up(0.2)
        t = H.bench_graph(lambda i: ops.dequant(qws[i]), reps=16, trials=args.trials)
        nb = H.dequant_bytes(K, N, args.group_size)
        gbps = H.achieved_gbps(nb, t.median_ms)
        row = {"bench": "dequant", "K": K, "N": N, "impl": "dequant fast",
               "us": round(t.median_ms * 1e3, 2), "GB/s": round(gbps),
               "%8TB/s": round(100 * gbps / H.HBM_PEAK_GBPS, 1),
               "%copy": round(100 * gbps / copy, 1), **_clock(t)}
        _emit(rows, row)
        del qws
        torch.cuda.empty_cache()


def crossover(args, rows):
    K, N = args.shape
    qws, gen = _weights(K, N, args.group_size, seed=7)
    w16 = _fp16_baseline(qws[0])
    for M in args.M or [1, 2, 4, 8, 9, 16, 24, 32, 33, 48, 64, 96, 128]:
        X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
        f = H.bench_graph(lambda i: torch.mm(X, w16[i]), reps=32, trials=args.trials)
        row = {"bench": "crossover", "M": M, "K": K, "N": N,
               "hipblaslt_fp16_us": round(f.median_ms * 1e3, 2)}
        if M <= ops.DECODE_MAX_M:
            _check(ops.gemv(X, qws[0]), X, qws[0], f"gemv M={M}")
            row["gemv_us"] = round(H.bench_graph(lambda i: ops.gemv(X, qws[i]), reps=32,
                                                 trials=args.trials).median_ms * 1e3, 2)
        _check(ops.gemm(X, qws[0]), X, qws[0], f"gemm M={M}")
        row["gemm_us"] = round(H.bench_graph(lambda i: ops.gemm(X, qws[i]), reps=32,
                                             trials=args.trials).median_ms * 1e3, 2)
        row["matmul_us"] = min(v for k, v in row.items() if k in ("gemv_us", "gemm_us"))
        row["vs_fp16"] = round(row["hipblaslt_fp16_us"] / row["matmul_us"], 2)
        _emit(rows, row)


def strips(args, rows):
    """What bounds one decode launch: the M = 1 GEMV at K = 4096 over N (one
    64-column strip per workgroup, one workgroup per CU up to 256 strips),
    then the streaming-read probe over the headline's bytes at a range of
    workgroup counts.  A time flat in the strip count means each CU streams
    its strip at a per-CU rate, whatever the others do."""
    K = 4096
    for N in args.N or [12288, 13312, 14336, 15360, 16384, 18432]:
        qws, gen = _weights(K, N, args.group_size, seed=K + N)
        X = torch.randn((1, K), generator=gen).to(torch.float16).cuda()
        _check(ops.gemv(X, qws[0]), X, qws[0], f"gemv 1x{K}x{N}")
        t = H.bench_graph(lambda i: ops.gemv(X, qws[i]), reps=64, trials=args.trials)
        nb = H.total_bytes(1, K, N, args.group_size, 4)
        us = t.median_ms * 1e3
        _emit(rows, {"bench": "strips", "what": "gemv M=1", "K": K, "N": N, "workgroups": N // 64,
                     "us": round(us, 2), "GB/s": round(nb / us / 1e3),
                     "GB/s per busy CU": round(nb / min(N // 64, 256) / us / 1e3, 2), **_clock(t)})
        del qws
        torch.cuda.empty_cache()
    fn = H._read_probe_fn()
    nb = H.total_bytes(1, 4096, 14336, args.group_size, 4)
    stride = (nb + 4095) // 4096 * 4096
    copies = (1 << 30) // stride + 4  # > 1 GiB in rotation: every read streams from HBM
    buf = torch.ones(stride * copies // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    for wgs in (224, 256, 512, 1024, 4096):
        def run(i):
            rc = fn(buf.data_ptr() + (i % copies) * stride, nb, wgs, sink.data_ptr(),
                    torch.cuda.current_stream().cuda_stream)
            if rc:
                raise RuntimeError(f"read probe failed ({rc})")
        t = H.bench_graph(run, reps=64, trials=args.trials)
        us = t.median_ms * 1e3
        _emit(rows, {"bench": "strips", "what": "read probe", "K": 4096, "N": 14336, "workgroups": wgs,
                     "us": round(us, 2), "GB/s": round(nb / us / 1e3),
                     "GB/s per busy CU": round(nb / min(wgs, 256) / us / 1e3, 2), **_clock(t)})
    del buf, sink
    torch.cuda.empty_cache()


LAUNCH_SHAPES = [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 8192)]


def launch(args, rows):
    """What launching costs: the same ``matmul`` calls eager and replayed from
    a HIP graph (reference bench/launch_overhead.py:32-58); the difference is
    per-call host work, which a captured decode step does not pay."""
    for K, N in LAUNCH_SHAPES:
        qws, gen = _weights(K, N, args.group_size, seed=K + N)
        for M in args.M or [1]:
            X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
            _check(ops.matmul(X, qws[0]), X, qws[0], f"matmul {M}x{K}x{N}")
            e = H.bench(lambda i: ops.matmul(X, qws[i]), reps=64, trials=args.trials)
            g = H.bench_graph(lambda i: ops.matmul(X, qws[i]), reps=64, trials=args.trials)
            nb = H.total_bytes(M, K, N, args.group_size, 4)
            _emit(rows, {"bench": "launch", "M": M, "K": K, "N": N,
                         "eager_us": round(e.median_ms * 1e3, 2),
                         "graph_us": round(g.median_ms * 1e3, 2),
                         "launch_us": round((e.median_ms - g.median_ms) * 1e3, 2),
                         "eager_GB/s": round(H.achieved_gbps(nb, e.median_ms)),
                         "graph_GB/s": round(H.achieved_gbps(nb, g.median_ms))})
        del qws
        torch.cuda.empty_cache()


def _attention_ref(qkv, kc, vc, pos, n_heads, n_kv, cos, sin):
    """fp32 attention of the token at ``pos`` over cache rows 0 .. pos - 1
    plus its own k (rotated, rounded to fp16 as the cache stores it) and v."""
    hd = 128
    q = qkv[0, :n_heads * hd].float().view(n_heads, hd)
    k = qkv[0, n_heads * hd:(n_heads + n_kv) * hd].float().view(n_kv, hd)
    v = qkv[0, (n_heads + n_kv) * hd:].float().view(n_kv, hd)
    c, s = cos[pos], sin[pos]

    def rot(x):
        lo, hi = x[:, :hd // 2], x[:, hd // 2:]
        return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=1)

    q, k = rot(q), rot(k).half().float()
    K = torch.cat([kc[:, :pos].float(), k[:, None]], dim=1).repeat_interleave(n_heads // n_kv, 0)
    V = torch.cat([vc[:, :pos].float(), v[:, None]], dim=1).repeat_interleave(n_heads // n_kv, 0)
    p = torch.softmax(torch.bmm(K.contiguous(), q[:, :, None].contiguous())[:, :, 0] / hd ** 0.5, -1)
    return torch.bmm(p[:, None, :].contiguous(), V.contiguous())[:, 0].reshape(1, -1)


def attention(args, rows):
    """The decode step's attention (Llama-3-8B: 32 query heads, 8 kv heads,
    head_dim 128, rotary) at several cache lengths, over 32 distinct caches
    as the 32 layers of a step would hold them; each position checked against
    an fp32 reference first."""
    from .glue import attention_bytes, attention_decode, rope_tables
    n_heads, n_kv, max_seq, layers = 32, 8, 4096, 32
    gen = torch.Generator().manual_seed(7)
    cos, sin = rope_tables(max_seq)
    kcs = [torch.randn((n_kv, max_seq, 128), generator=gen).half().cuda() for _ in range(layers)]
    vcs = [torch.randn((n_kv, max_seq, 128), generator=gen).half().cuda() for _ in range(layers)]
    qkv = torch.randn((1, (n_heads + 2 * n_kv) * 128), generator=gen).half().cuda()
    for pos in args.pos:
        ref = _attention_ref(qkv, kcs[0], vcs[0], pos, n_heads, n_kv, cos, sin)
        y = attention_decode(qkv, kcs[0], vcs[0], pos, (cos, sin))
        err = float((y.float() - ref).abs().max() / ref.pow(2).mean().sqrt())
        if not err <= TOL:
            raise RuntimeError(f"attention pos={pos}: max|y - ref| = {err:.3e} * rms(ref)")
        t = H.bench_graph(lambda i: attention_decode(qkv, kcs[i % layers], vcs[i % layers], pos,
                                                     (cos, sin)), reps=32, trials=args.trials)
        _emit(rows, {"bench": "attention", "pos": pos, "chunks": (pos + 128) // 128,
                     "us": round(t.median_ms * 1e3, 2),
                     "kv_GB/s": round(H.achieved_gbps(attention_bytes(n_kv, pos), t.median_ms)),
                     "max_err_rms": float(f"{err:.2e}"), **_clock(t)})


def autotune(args, rows):
    """The GEMV's launch geometry swept over K splits x workgroup size, each
    point checked first, against the built-in plan (reference
    bench/autotune.py:30-72).  ``vs_plan`` > 1 means the point beats the plan."""
    for K, N in LAUNCH_SHAPES + [(4096, 1024)]:
        qws, gen = _weights(K, N, args.group_size, seed=K + N)
        groups = K // args.group_size
        for M in args.M or [1]:
            X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
            plan = H.bench_graph(lambda i: ops.gemv(X, qws[i]), reps=32, trials=args.trials)
            for threads in (64, 128, 256, 512, 1024):
                for splits in (1, 2, 4, 8, 16):
                    if splits > groups:
                        continue
                    try:
                        y = ops.gemv(X, qws[0], 4, splits, threads)
                    except RuntimeError:  # geometry the kernel does not take at this M
                        continue
                    err = _check(y, X, qws[0], f"gemv {M}x{K}x{N} s={splits} t={threads}")
                    t = H.bench_graph(lambda i: ops.gemv(X, qws[i], 4, splits, threads),
                                      reps=32, trials=args.trials)
                    nb = H.total_bytes(M, K, N, args.group_size, 4)
                    _emit(rows, {"bench": "autotune", "M": M, "K": K, "N": N,
                                 "threads": threads, "splits": splits,
                                 "us": round(t.median_ms * 1e3, 2),
                                 "GB/s": round(H.achieved_gbps(nb, t.median_ms)),
                                 "plan_us": round(plan.median_ms * 1e3, 2),
                                 "vs_plan": round(plan.median_ms / t.median_ms, 2),
                                 "max_err_rms": float(f"{err:.2e}")})
        del qws
        torch.cuda.empty_cache()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("what", choices=["decode", "prefill", "dequant", "crossover", "launch",
                                     "autotune", "attention", "strips"])
    ap.add_argument("--N", type=int, nargs="*", help="strips: the weight widths (K = 4096)")
    ap.add_argument("--M", type=int, nargs="*", help="batch sizes (default: the benchmark shapes)")
    ap.add_argument("--pos", type=int, nargs="*", default=[0, 127, 128, 511, 1023, 2047, 4095],
                    help="attention: cache positions of the decoded token")
    ap.add_argument("--shape", type=int, nargs=2, metavar=("K", "N"), default=[4096, 14336],
                    help="crossover: the weight shape (default 4096 14336)")
    ap.add_argument("--group-size", type=int, default=128)
    ap.add_argument("--trials", type=int, default=10)
    ap.add_argument("--markdown", action="store_true")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("bench_shapes needs a GPU", file=sys.stderr)
        return 1
    ops.extension()
    torch.backends.cuda.matmul.allow_tf32 = False
    print(f"# {H.device_summary()}", file=sys.stderr, flush=True)
    rows = []
    {"decode": decode, "prefill": prefill, "dequant": dequant, "crossover": crossover,
     "launch": launch, "autotune": autotune, "attention": attention,
     "strips": strips}[args.what](args, rows)
    if args.markdown and rows:
        cols = [k for k in rows[0] if k != "bench"]
        print(H.markdown_table(rows, cols), file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
