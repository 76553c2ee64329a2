"""Writes the committed golden vectors in this directory.

The vectors are produced by the CPU oracle (``oracle/``), itself pinned by the
known-answer and closed-form checks in ``tests/test_oracle.py``.  They freeze
seeded inputs and the reference path's outputs -- dequantized weights
(bit-exact) and fp32-accumulated matmul results -- so GPU tests can compare
against stored data and CPU tests can detect any drift in the oracle.

Inputs follow the benchmark's synthetic distributions: nibbles uniform in
[0, 15], scales fp16(U(0.002, 0.02)), activations fp16(N(0, 1)); plus the
reference's dequant sweep (tests/test_dequant.py:27-44 in arvindcr4/nibblegemm):
every value in every slot on a 0xF background, all slots equal, random words.

Run: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402

# (name, M, K, N, group_size, seed)
MATMUL_CASES = [
    ("m1_k256_n132_g128", 1, 256, 132, 128, 11),
    ("m3_k256_n256_g64", 3, 256, 256, 64, 12),
    ("m8_k512_n260_g128", 8, 512, 260, 128, 13),
    ("m17_k256_n132_g64", 17, 256, 132, 64, 14),
    ("m65_k512_n256_g128", 65, 512, 256, 128, 15),
]


def sweep_nibbles(K: int, extra_cols: int, seed: int) -> np.ndarray:
    k_off = np.arange(K) % 8
    slot, value = np.divmod(np.arange(128), 16)
    isolated = np.where(k_off[:, None] == slot[None, :], value[None, :], 15)
    uniform = np.tile(np.arange(16), (K, 1))
    rand = np.random.default_rng(seed).integers(0, 16, size=(K, extra_cols))
    return np.concatenate([isolated, uniform, rand], axis=1).astype(np.uint8)


def main() -> None:
    out = {}
    for name, M, K, N, g, seed in MATMUL_CASES:
        X, packed, scales = O.synthetic_case(M, K, N, g, seed)
        W = O.dequantize(packed, scales, K, g)
        Y = O.matmul_f16w(X, W)
        out[f"{name}/X"] = X.view(np.uint16)
        out[f"{name}/qweight"] = packed
        out[f"{name}/scales"] = scales.view(np.uint16)
        if M == 1:  # keep one dense dequant output among the matmul cases
            out[f"{name}/W"] = W.view(np.uint16)
        out[f"{name}/Y"] = Y.view(np.uint16)
        out[f"{name}/meta"] = np.array([M, K, N, g, seed], dtype=np.int64)

    # dequant sweep with scales spanning 2^-10 .. 2^10 (all-normal products)
    qu = sweep_nibbles(256, 116, seed=1)
    rng = np.random.default_rng(2)
    for g in (64, 128):
        rows = 256 // g
        s = (2.0 ** rng.uniform(-10.0, 10.0, size=(rows, qu.shape[1]))).astype(np.float32)
        s[0, :4] = [2.0 ** -10, 2.0 ** 10, 1.0, 2.0 ** -3]
        s16 = O.f32_to_f16(s)
        packed = O.pack_nibbles(qu)
        W = O.dequantize(packed, s16, 256, g)
        out[f"sweep_g{g}/qweight"] = packed
        out[f"sweep_g{g}/scales"] = s16.view(np.uint16)
        out[f"sweep_g{g}/W"] = W.view(np.uint16)
        out[f"sweep_g{g}/meta"] = np.array([256, qu.shape[1], g], dtype=np.int64)

    path = os.path.join(HERE, "w4a16_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
