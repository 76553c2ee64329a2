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

``fp16mm`` is the baseline the prefill GEMM is compared with: ``torch.mm``
(hipBLASLt) on fp16 weights of the same shape, rotated the same way.
``copy`` is the calibration kernel for the HBM byte counters: a device copy
of a known size (reads and writes ``--mib`` MiB each), so FETCH_SIZE and
WRITE_SIZE per dispatch can be scaled to bytes.  The weights of gemv,
dequant and gemm rotate through copies spanning >= 1 GiB, so each call
streams them from HBM rather than from the 256 MiB Infinity Cache.
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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("kernel", choices=["gemv", "gemm", "dequant", "copy", "fp16mm"])
    ap.add_argument("--M", type=int, default=1)
    ap.add_argument("--K", type=int, default=4096)
    ap.add_argument("--N", type=int, default=14336)
    ap.add_argument("--G", type=int, default=128)
    ap.add_argument("--calls", type=int, default=50)
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--version", type=int, default=6, choices=[6, 7], help="gemm version")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("profile_target needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    ops.extension()
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
