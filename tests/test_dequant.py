"""Bit-exactness of the HIP dequant kernel (reference tests/test_dequant.py).

Every assertion is ``array_equal`` on fp16 bit patterns, never a tolerance:
the magic-exponent path builds the exact n - 8 and rounds (n - 8) * s once in
v_pk_mul_f16; the scalar path forms the exact product in fp32 and rounds once
on conversion; the oracle does the same in C.  All three round the same real
number once, so any difference is a wrong mask, bias, slot or group index.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from cases import to_dev_qw

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w4a16_golden.npz")


def sweep_nibbles(K: int = 128, extra_cols: int = 116, seed: int = 0) -> np.ndarray:
    """reference tests/test_dequant.py:27-44"""
    k_off = np.arange(K) % 8
    slot, value = np.divmod(np.arange(128), 16)
    isolated = np.where(k_off[:, None] == slot[None, :], value[None, :], 15)
    uniform = np.tile(np.arange(16), (K, 1))
    rand = np.random.default_rng(seed).integers(0, 16, size=(K, extra_cols))
    return np.concatenate([isolated, uniform, rand], axis=1).astype(np.uint8)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def assert_all_agree(oracle, qu: np.ndarray, scales_f32: np.ndarray, g: int) -> np.ndarray:
    K, N = qu.shape
    packed = oracle.pack_nibbles(qu)
    s16 = oracle.f32_to_f16(scales_f32)
    qw = to_dev_qw(packed, s16, K, N, g)
    fast = ng.dequant(qw, fast=True)
    slow = ng.dequant(qw, fast=False)
    ref = oracle.dequantize(packed, s16, K, g)
    assert fast.shape == (K, N) and fast.dtype == torch.float16
    assert np.array_equal(bits(fast), bits(slow)), "magic decode disagrees with the scalar decode"
    assert np.array_equal(bits(fast), ref.view(np.uint16)), "kernel disagrees with the oracle"
    host = ng.dequantize(qw)  # the package's host decode
    assert np.array_equal(host.numpy().view(np.uint16), ref.view(np.uint16))
    return fast.float().cpu().numpy()


@pytest.mark.parametrize("group_size", [64, 128])
def test_decode_bit_exact_unit_scales(oracle, group_size):
    qu = sweep_nibbles(K=128)
    scales = np.ones((qu.shape[0] // group_size, qu.shape[1]), dtype=np.float32)
    fast = assert_all_agree(oracle, qu, scales, group_size)
    assert fast.min() == -8.0 and fast.max() == 7.0


@pytest.mark.parametrize("group_size", [64, 128])
def test_decode_bit_exact_varied_scales(oracle, group_size):
    qu = sweep_nibbles(K=256, seed=1)
    rows, N = qu.shape[0] // group_size, qu.shape[1]
    rng = np.random.default_rng(2)
    scales = (2.0 ** rng.uniform(-10.0, 10.0, size=(rows, N))).astype(np.float32)
    scales[0, :4] = [2.0 ** -10, 2.0 ** 10, 1.0, 2.0 ** -3]
    assert_all_agree(oracle, qu, scales, group_size)


@pytest.mark.parametrize("group_size", [64, 128])
def test_decode_subnormal_and_overflowing_products(oracle, group_size):
    """Products below fp16's normal range and above its max: all three paths
    must round into subnormals / to inf identically (fp16 denormals kept)."""
    qu = sweep_nibbles(K=256, seed=7)
    rows, N = qu.shape[0] // group_size, qu.shape[1]
    rng = np.random.default_rng(8)
    scales = (2.0 ** rng.uniform(-24.0, 15.9, size=(rows, N))).astype(np.float32)
    assert_all_agree(oracle, qu, scales, group_size)


@pytest.mark.parametrize("group_size", [64, 128])
def test_decoded_values_stay_within_the_codebook_range(oracle, group_size):
    qu = sweep_nibbles(K=256, seed=3)
    rows, N = qu.shape[0] // group_size, qu.shape[1]
    rng = np.random.default_rng(4)
    scales = (2.0 ** rng.uniform(-6.0, 6.0, size=(rows, N))).astype(np.float32)
    out = assert_all_agree(oracle, qu, scales, group_size).astype(np.float64)
    s = np.repeat(oracle.f32_to_f16(scales).astype(np.float64), group_size, axis=0)
    slack = 1.0 + 2.0 ** -11
    assert np.all(out <= 7.0 * s * slack) and np.all(out >= -8.0 * s * slack)


@pytest.mark.parametrize("group_size", [64, 128])
def test_scales_are_applied_per_group(oracle, group_size):
    qu = sweep_nibbles(K=512, extra_cols=4, seed=5)
    rows, N = qu.shape[0] // group_size, qu.shape[1]
    scales = np.repeat((2.0 ** np.arange(rows, dtype=np.float32))[:, None], N, axis=1)
    assert_all_agree(oracle, qu, scales, group_size)


@pytest.mark.parametrize("K,N", [(64, 1), (64, 3), (128, 6), (256, 12), (128, 8), (256, 1000),
                                 (512, 2052)])
def test_ragged_widths(oracle, K, N):
    """N not a multiple of 8 (4-column and 1-column kernel variants)."""
    rng = np.random.default_rng(K + N)
    qu = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    scales = rng.uniform(0.002, 0.02, size=(K // 64, N)).astype(np.float32)
    assert_all_agree(oracle, qu, scales, 64)


def test_empty_weight():
    qw = ng.QuantizedWeight(torch.zeros((0, 16), dtype=torch.int32, device="cuda"),
                            torch.zeros((0, 16), dtype=torch.float16, device="cuda"), 128, 0, 16)
    assert ng.dequant(qw).shape == (0, 16)


def test_golden_sweep_vectors():
    z = np.load(GOLDEN)
    for g in (64, 128):
        K, N, gg = z[f"sweep_g{g}/meta"].tolist()
        qw = to_dev_qw(z[f"sweep_g{g}/qweight"], z[f"sweep_g{g}/scales"], K, N, gg)
        assert np.array_equal(bits(ng.dequant(qw, fast=True)), z[f"sweep_g{g}/W"])
        assert np.array_equal(bits(ng.dequant(qw, fast=False)), z[f"sweep_g{g}/W"])


def test_full_size_gate_up_bit_exact(oracle):
    """The headline shape 4096 x 14336 at the benchmark distributions."""
    K, N, g = 4096, 14336, 128
    _, packed, scales = oracle.synthetic_case(1, K, N, g, seed=21)
    qw = to_dev_qw(packed, scales, K, N, g)
    ref = oracle.dequantize(packed, scales, K, g)
    out = ng.dequant(qw)
    assert np.array_equal(bits(out), ref.view(np.uint16))
