"""Seeded inputs shared by the GPU parity tests.

Every case is generated once on the host (numpy), then copied to the GPU, so
the HIP kernels and the CPU oracle see the same bytes.
"""
from __future__ import annotations

import numpy as np
import torch

import nibblegemm_amd as ng
import oracle as O

#: The decode benchmark shapes: M = 1, g = 128.
DECODE_SHAPES = [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 8192), (4096, 1024)]


def to_dev_qw(packed: np.ndarray, scales: np.ndarray, K: int, N: int, g: int,
              device="cuda") -> ng.QuantizedWeight:
    return ng.QuantizedWeight(
        torch.from_numpy(np.ascontiguousarray(packed).view(np.int32)).to(device),
        torch.from_numpy(np.ascontiguousarray(scales).view(np.float16)).to(device),
        g, K, N)


def synthetic(M: int, K: int, N: int, g: int = 128, seed: int = 0):
    """The benchmark distributions: returns (X_np fp16, packed, scales fp16, X_dev, qw_dev)."""
    X, packed, scales = O.synthetic_case(M, K, N, g, seed)
    Xd = torch.from_numpy(X.copy()).to("cuda")
    return X, packed, scales, Xd, to_dev_qw(packed, scales, K, N, g)


def quantized(M: int, K: int, N: int, g: int, seed: int = 0):
    """The reference tests' cases: W = randn * 0.02 quantised with RTN,
    X = randn (tests/test_gemv.py:32-37 in arvindcr4/nibblegemm)."""
    gen = torch.Generator().manual_seed(seed)
    W = torch.randn(K, N, generator=gen) * 0.02
    qw = ng.quantize(W, group_size=g)
    X = torch.randn(M, K, generator=gen).to(torch.float16)
    return X.numpy(), qw.qweight.numpy(), qw.scales.numpy(), X.to("cuda"), qw.to("cuda")


def oracle_y(X: np.ndarray, packed: np.ndarray, scales: np.ndarray, K: int, g: int) -> np.ndarray:
    """The reference path on the host: dequantize, fp32 matmul, fp16."""
    return O.reference_matmul(X, packed, scales, K, g).astype(np.float32)


def oracle_y_rows(X: np.ndarray, rows, packed, scales, K: int, g: int) -> np.ndarray:
    """Reference rows ``rows`` only (for prefill shapes too large to do whole)."""
    return O.reference_matmul(np.ascontiguousarray(X[rows]), packed, scales, K, g).astype(np.float32)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rms_err(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / np.sqrt(np.mean(ref * ref)))


def rel_err(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / np.abs(ref).mean())
