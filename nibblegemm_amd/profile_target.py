"""Minimal driver for a profiler (the role of the reference's
scripts/profile_target.py:15-36): runs one kernel a fixed number of times on
cuda:0 and nothing else, so ``rocprofv3 --kernel-trace`` / ``--pmc`` output
holds only that kernel (plus setup copies).

    python3 -m nibblegemm_amd.profile_target gemv --K 4096 --N 14336 --M 1 --calls 50
    python3 -m nibblegemm_amd.profile_target dequant --K 4096 --N 14336 --calls 20
    python3 -m nibblegemm_amd.profile_target gemm --M 2048 --K 4096 --N 14336 --calls 10
    python3 -m nibblegemm_amd.profile_target gemm --M 4096 --K 14336 --N 4096 --version 7
    python3 -m nibblegemm_amd.profile_target copy --mib 256 --calls 20
    python3 -m nibblegemm_amd.profile_target fp16mm --M 2048 --K 4096 --N 14336 --calls 10
    python3 -m nibblegemm_amd.profile_target gemv-timeline --K 4096 --N 14336 --calls 300 --trials 30

``fp16mm`` is the baseline the prefill GEMM is compared with: ``torch.mm``
(hipBLASLt) on fp16 weights of the same shape, rotated the same way.
``copy`` is the calibration kernel for the HBM byte counters: a device copy
of a known size (reads and writes ``--mib`` MiB each), so FETCH_SIZE and
WRITE_SIZE per dispatch can be scaled to bytes.  The weights of gemv,
dequant and gemm rotate through copies spanning >= 1 GiB, so each call
streams them from HBM rather than from the 256 MiB Infinity Cache.

``gemv-timeline`` reads the decode GEMV's in-kernel timeline
(``nibble_gemv_timeline``): per trial it issues ``--calls`` back-to-back M = 1
calls and keeps the last one's per-wave timestamps, then prints where a
workgroup's time goes (phase medians over workgroups, then over trials), the
spread of workgroup starts and ends, and the mean time of each strip.
"""
from __future__ import annotations

import argparse
import sys

import torch

from . import harness as H
from . import ops
from .quant import QuantizedWeight, pack_nibbles


def _weights(K: int, N: int, G: int, dev):
    gen = torch.Generator().manual_seed(0)
    qu = torch.randint(0, 16, (K, N), generator=gen, dtype=torch.uint8).numpy()
    qweight = torch.from_numpy(pack_nibbles(qu)).to(dev)
    scales = (torch.rand((K // G, N), generator=gen) * 0.018 + 0.002).to(torch.float16).to(dev)
    return H.weight_ring(QuantizedWeight(qweight, scales, G, K, N)), gen


# Phases of a workgroup, between the timeline's points (the latest wave of
# the workgroup at each point).
_PHASES = [("prologue issue", 0, 1), ("copies land", 1, 2), ("first group", 2, 3),
           ("other groups", 3, 4), ("partials", 4, 5), ("sum and stores", 5, 6)]


def _gemv_timeline(args, dev) -> int:
    import numpy as np  # noqa: PLC0415

    qws, gen = _weights(args.K, args.N, args.G, dev)
    X = torch.randn((1, args.K), generator=gen).to(torch.float16).to(dev)
    ext = ops.extension()
    # Room for any strip plan: 16-column strips, 16 waves.
    strips16 = -(-args.N // 16)
    grid = 8 * -(-strips16 // 8)
    stamps = torch.zeros(grid * 16 * 8, dtype=torch.int64, device=dev)
    rows, ends = [], []
    if ext.gemv_timeline(stamps.data_ptr(), stamps.numel() * 8) != 0:
        raise RuntimeError(ext.last_error())
    try:
        for i in range(200):
            ops.gemv(X, qws[i % len(qws)])
        for trial in range(args.trials):
            stamps.zero_()
            for i in range(args.calls):
                ops.gemv(X, qws[(trial * 7 + i) % len(qws)])
            torch.cuda.synchronize()
            t = stamps.view(-1, 8).cpu().numpy()
            t = t[t[:, 0] > 0]
            if len(t) == 0:
                raise RuntimeError("no timeline written: this shape's M = 1 plan is not the strip kernel")
            wg = (t[:, 7] >> 40).astype(np.int64)
            ids = np.unique(wg)
            start = np.array([t[wg == b, 0].min() for b in ids])
            late = np.array([t[wg == b, :7].max(axis=0) for b in ids])  # latest wave per point
            t0 = start.min()
            us = lambda v: (v.astype(np.float64)) * 0.01  # noqa: E731 (100 MHz ticks)
            row = {name: float(np.median(us(late[:, b] - (start if a == 0 else late[:, a]))))
                   for name, a, b in _PHASES}
            row["workgroup"] = float(np.median(us(late[:, 6] - start)))
            row["slowest workgroup"] = float(us(late[:, 6] - start).max())
            row["start spread"] = float(us(start - t0).max())
            row["span"] = float(us(late[:, 6].max() - t0))
            rows.append(row)
            ends.append(dict(zip(ids.tolist(), us(late[:, 6] - start).tolist())))
    finally:
        ext.gemv_timeline(None, 0)
    keys = list(rows[0])
    print(f"gemv-timeline M=1 K={args.K} N={args.N} g={args.G}: {len(ends[0])} workgroups, the last "
          f"of {args.calls} back-to-back calls in each of {args.trials} trials; us")
    print("| statistic | " + " | ".join(keys) + " |")
    print("|---|" + "---|" * len(keys))
    for name, f in (("median", np.median), ("min", np.min), ("max", np.max)):
        print(f"| {name} over trials | " + " | ".join(f"{f([r[k] for r in rows]):.2f}" for k in keys) + " |")
    ids = sorted(ends[0])
    mean = {b: float(np.mean([e[b] for e in ends if b in e])) for b in ids}
    med = float(np.median(list(mean.values())))
    slow = sorted((b for b in ids if mean[b] > med + 0.25), key=lambda b: -mean[b])
    spx = len(ids) // 8  # strips per XCD: workgroup b runs strip (b % 8) * spx + b // 8
    print(f"workgroups more than 0.25 us above the median ({med:.2f} us), mean over trials: "
          + ", ".join(f"b{b} (strip {(b % 8) * spx + b // 8}): {mean[b]:.2f}" for b in slow))
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("kernel", choices=["gemv", "gemm", "dequant", "copy", "fp16mm", "gemv-timeline"])
    ap.add_argument("--M", type=int, default=1)
    ap.add_argument("--K", type=int, default=4096)
    ap.add_argument("--N", type=int, default=14336)
    ap.add_argument("--G", type=int, default=128)
    ap.add_argument("--calls", type=int, default=50)
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--version", type=int, default=6, choices=[6, 7], help="gemm version")
    ap.add_argument("--trials", type=int, default=30, help="gemv-timeline: timelines kept")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("profile_target needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    ops.extension()
    if args.kernel == "gemv-timeline":
        return _gemv_timeline(args, dev)
    if args.kernel == "copy":
        n = args.mib * (1 << 20) // 2
        src = torch.ones(n, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(args.calls):
            dst.copy_(src)
    elif args.kernel == "fp16mm":
        qws, gen = _weights(args.K, args.N, args.G, dev)
        X = torch.randn((args.M, args.K), generator=gen).to(torch.float16).to(dev)
        w16 = H.tensor_ring(ops.dequant(qws[0]))
        torch.backends.cuda.matmul.allow_tf32 = False
        torch.cuda.synchronize()
        for i in range(args.calls):
            torch.mm(X, w16[i])
    else:
        qws, gen = _weights(args.K, args.N, args.G, dev)
        X = torch.randn((args.M, args.K), generator=gen).to(torch.float16).to(dev)
        fn = {"gemv": lambda i: ops.gemv(X, qws[i]),
              "gemm": lambda i: ops.gemm(X, qws[i], version=args.version),
              "dequant": lambda i: ops.dequant(qws[i])}[args.kernel]
        torch.cuda.synchronize()
        for i in range(args.calls):
            fn(i)
    torch.cuda.synchronize()
    print(f"profile_target {args.kernel}: {args.calls} calls done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
