"""CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker.  The shipped package
(``nibblegemm_amd``) never imports it and has no CPU fallback onto it.

Thin ``ctypes`` front end over ``nibble_oracle.c`` (a plain-C restatement of
``python/nibblegemm/quant.py:48-215`` in the reference), operating on numpy
arrays.  fp16 data crosses the boundary as ``uint16`` bit patterns so that no
numpy or torch conversion sits between the C code and the bytes it produced.

Reference lines each function follows:

=====================  ==============================================
``pack_nibbles``       python/nibblegemm/quant.py:164-182
``unpack_nibbles``     python/nibblegemm/quant.py:185-196
``quantize_rtn``       python/nibblegemm/quant.py:127-161 (clip_search=False)
``dequantize``         python/nibblegemm/quant.py:199-204
``reference_matmul``   python/nibblegemm/quant.py:207-215
``matmul_f64``         brute-force double-precision product (no counterpart)
``rel_err``            tests/conftest.py:69-82
``rms_err``            the north-star metric: max|y-ref| / rms(ref)
=====================  ==============================================

How each one is pinned is listed in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import time

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libnibble_oracle.so")
_lib = None

SLOT_FOR_K = (0, 4, 1, 5, 2, 6, 3, 7)
ZERO_POINT = 8
PACK_FACTOR = 8


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.nibble_oracle_f16_to_f32.restype = ctypes.c_float
        L.nibble_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.nibble_oracle_f32_to_f16.restype = ctypes.c_uint16
        L.nibble_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.nibble_oracle_f32_to_f16_array.argtypes = [p, p, i64]
        L.nibble_oracle_f16_to_f32_array.argtypes = [p, p, i64]
        L.nibble_oracle_pack.restype = ctypes.c_int
        L.nibble_oracle_pack.argtypes = [p, i64, i64, p]
        L.nibble_oracle_unpack.argtypes = [p, i64, i64, p]
        L.nibble_oracle_quantize_rtn.restype = ctypes.c_int
        L.nibble_oracle_quantize_rtn.argtypes = [p, i64, i64, i64, p, p, p]
        L.nibble_oracle_dequantize.argtypes = [p, p, i64, i64, i64, p]
        L.nibble_oracle_matmul_f32.argtypes = [p, p, i64, i64, i64, p, p]
        L.nibble_oracle_matmul_f64.argtypes = [p, p, i64, i64, i64, p]
        L.nibble_oracle_max_threads.restype = ctypes.c_int
        L.nibble_oracle_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _as_u16(a) -> np.ndarray:
    """fp16 data as its uint16 bit pattern (accepts float16 or uint16 arrays)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


# --------------------------------------------------------------------------
# binary16
# --------------------------------------------------------------------------
def f32_to_f16(x) -> np.ndarray:
    """RNE narrowing; returns float16 array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().nibble_oracle_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f16_to_f32(h) -> np.ndarray:
    h = _as_u16(h)
    out = np.empty(h.shape, dtype=np.float32)
    lib().nibble_oracle_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


# --------------------------------------------------------------------------
# format
# --------------------------------------------------------------------------
def pack_nibbles(qu: np.ndarray) -> np.ndarray:
    """uint8 [K, N] in [0,15] -> int32 [K/8, N] (quant.py:164-182)."""
    qu = np.ascontiguousarray(qu, dtype=np.uint8)
    K, N = qu.shape
    out = np.empty((max(K // 8, 0), N), dtype=np.uint32)
    rc = lib().nibble_oracle_pack(_ptr(qu), K, N, _ptr(out))
    if rc == -1:
        raise ValueError(f"K={K} must be divisible by 8")
    if rc == -2:
        raise ValueError("quantised values must fit in 4 bits")
    return out.view(np.int32)


def unpack_nibbles(packed: np.ndarray, K: int) -> np.ndarray:
    """int32 [K/8, N] -> uint8 [K, N] (quant.py:185-196)."""
    p = np.ascontiguousarray(packed).view(np.uint32)
    rows, N = p.shape
    if rows * 8 != K:
        raise ValueError(f"packed rows={rows} inconsistent with K={K}")
    out = np.empty((K, N), dtype=np.uint8)
    lib().nibble_oracle_unpack(_ptr(p), rows, N, _ptr(out))
    return out


def quantize_rtn(W: np.ndarray, group_size: int = 128):
    """fp32 [K, N] -> (qu uint8 [K,N], scales_f32 [K/G,N], scales fp16 [K/G,N])."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    K, N = W.shape
    qu = np.empty((K, N), dtype=np.uint8)
    rows = K // group_size if group_size > 0 else 0
    s32 = np.empty((rows, N), dtype=np.float32)
    s16 = np.empty((rows, N), dtype=np.uint16)
    rc = lib().nibble_oracle_quantize_rtn(_ptr(W), K, N, group_size, _ptr(qu), _ptr(s32), _ptr(s16))
    if rc != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}, itself a multiple of 8")
    return qu, s32, s16.view(np.float16)


def dequantize(packed: np.ndarray, scales, K: int, group_size: int) -> np.ndarray:
    """fp16 [K, N] = f16((nibble-8) * f32(scale)) (quant.py:199-204)."""
    p = np.ascontiguousarray(packed).view(np.uint32)
    s = _as_u16(scales)
    rows, N = p.shape
    assert rows * 8 == K and s.shape == (K // group_size, N)
    out = np.empty((K, N), dtype=np.uint16)
    lib().nibble_oracle_dequantize(_ptr(p), _ptr(s), K, N, group_size, _ptr(out))
    return out.view(np.float16)


def matmul_f16w(X, W, want_f32: bool = False):
    """f16(X_f32 @ W_f32) with fp32 accumulation; X [M,K] fp16, W [K,N] fp16."""
    x = _as_u16(X)
    w = _as_u16(W)
    M, K = x.shape
    K2, N = w.shape
    assert K == K2
    y = np.empty((M, N), dtype=np.uint16)
    yf = np.empty((M, N), dtype=np.float32) if want_f32 else None
    lib().nibble_oracle_matmul_f32(_ptr(x), _ptr(w), M, K, N, _ptr(y),
                                   _ptr(yf) if yf is not None else None)
    return (y.view(np.float16), yf) if want_f32 else y.view(np.float16)


def matmul_f64(X, W) -> np.ndarray:
    x = _as_u16(X)
    w = _as_u16(W)
    M, K = x.shape
    _, N = w.shape
    y = np.empty((M, N), dtype=np.float64)
    lib().nibble_oracle_matmul_f64(_ptr(x), _ptr(w), M, K, N, _ptr(y))
    return y


def reference_matmul(X, packed, scales, K: int, group_size: int) -> np.ndarray:
    """The reference's parity target: dequantize, then fp32 matmul, then fp16
    (quant.py:207-215)."""
    return matmul_f16w(X, dequantize(packed, scales, K, group_size))


# --------------------------------------------------------------------------
# metrics
# --------------------------------------------------------------------------
def rel_err(y, ref) -> float:
    """max|y-ref| / mean|ref| (tests/conftest.py:69-82)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / np.abs(ref).mean())


def rms_err(y, ref) -> float:
    """max|y-ref| / rms(ref): the north-star bound is rms_err <= 1e-2."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / np.sqrt(np.mean(ref * ref)))


# --------------------------------------------------------------------------
# seeded synthetic inputs (the benchmark distributions)
# --------------------------------------------------------------------------
def synthetic_case(M: int, K: int, N: int, group_size: int = 128, seed: int = 0):
    """Nibbles U{0..15}, scales fp16(U(0.002, 0.02)), X fp16(N(0,1)).

    Returns (X fp16 [M,K], packed int32 [K/8,N], scales fp16 [K/G,N]).
    """
    rng = np.random.default_rng(seed)
    qu = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    scales = f32_to_f16(rng.uniform(0.002, 0.02, size=(K // group_size, N)).astype(np.float32))
    X = f32_to_f16(rng.standard_normal(size=(M, K)).astype(np.float32))
    return X, pack_nibbles(qu), scales


# --------------------------------------------------------------------------
# CPU baseline timing (reported only)
# --------------------------------------------------------------------------
def time_reference_path(M: int, K: int, N: int, group_size: int = 128, reps: int = 5,
                        threads: int = 0, seed: int = 0, max_rows: int = 0) -> dict:
    """Time dequantize + reference matmul on this host's cores (median of reps).

    ``max_rows`` > 0 bounds the sample: the matmul runs on the first
    ``min(M, max_rows)`` rows of X and its time is scaled by M / rows (the
    fp32 product's work is linear in M; the dequantize runs whole).  The
    result says how many rows were timed."""
    L = lib()
    if threads > 0:
        L.nibble_oracle_set_threads(threads)
    rows = M if max_rows <= 0 else min(M, max_rows)
    X, packed, scales = synthetic_case(rows, K, N, group_size, seed)
    p = np.ascontiguousarray(packed).view(np.uint32)
    s = _as_u16(scales)
    x = _as_u16(X)
    W = np.empty((K, N), dtype=np.uint16)
    Y = np.empty((rows, N), dtype=np.uint16)
    dq, mm = [], []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        L.nibble_oracle_dequantize(_ptr(p), _ptr(s), K, N, group_size, _ptr(W))
        t1 = time.perf_counter()
        L.nibble_oracle_matmul_f32(_ptr(x), _ptr(W), rows, K, N, _ptr(Y), None)
        t2 = time.perf_counter()
        dq.append(t1 - t0)
        mm.append((t2 - t1) * M / rows)
    dq, mm = sorted(dq[1:]), sorted(mm[1:])
    tot = sorted(a + b for a, b in zip(dq, mm))
    return {
        "dequant_s": dq[len(dq) // 2],
        "matmul_s": mm[len(mm) // 2],
        "total_s": tot[len(tot) // 2],
        "threads": L.nibble_oracle_max_threads(),
        "reps": reps,
        "rows_timed": rows,
    }
