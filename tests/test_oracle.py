"""Pins the CPU oracle (oracle/nibble_oracle.c) to things other than itself.

Each function of the oracle is checked against the reference's own literal
known-answer tests, against closed forms the mathematics fixes, against an
independent library routine (numpy's IEEE binary16 conversion, integer
matmul), or by brute force on small inputs -- chosen so that a plausible slip
(a wrong slot, a dropped zero-point, a transposed operand, round-half-up
instead of half-even, a wrong group index) fails at least one of them.

| oracle function         | pinned by                                               |
|-------------------------|---------------------------------------------------------|
| pack / unpack           | literal slot table and word 0x75316420 (reference       |
|                         | tests/test_pack.py:17, :42); per-slot bit positions;    |
|                         | involution; the package's numpy packer                  |
| f32<->f16               | numpy float16 conversion, exhaustively / on every tie   |
| dequantize              | closed forms: unit scales give n-8, power-of-two scales |
|                         | give (n-8)*2^e exactly; numpy fp32 product + RNE; the   |
|                         | reference's codebook bound and per-group-scale checks   |
|                         | (tests/test_dequant.py:73-123)                          |
| quantize_rtn            | exact power-of-two cases, half-even ties, the nearest-  |
|                         | level property on random data, zero groups; the         |
|                         | package's torch quantizer bit-for-bit                   |
| matmul_f32 / f64        | exact integer matmul, a float64 bound                   |
| golden fixtures         | regenerated bit-for-bit (drift check)                   |
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng

#: Literal, not read from any module (reference tests/test_pack.py:17).
EXPECTED_SLOT_FOR_K = [0, 4, 1, 5, 2, 6, 3, 7]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w4a16_golden.npz")


def sweep_nibbles(K: int = 128, extra_cols: int = 116, seed: int = 0) -> np.ndarray:
    """Every nibble value in every slot on a 0xF background, all slots equal,
    then random words (reference tests/test_dequant.py:27-44)."""
    k_off = np.arange(K) % 8
    slot, value = np.divmod(np.arange(128), 16)
    isolated = np.where(k_off[:, None] == slot[None, :], value[None, :], 15)
    uniform = np.tile(np.arange(16), (K, 1))
    rand = np.random.default_rng(seed).integers(0, 16, size=(K, extra_cols))
    return np.concatenate([isolated, uniform, rand], axis=1).astype(np.uint8)


# --------------------------------------------------------------------------
# format
# --------------------------------------------------------------------------
def test_slot_table_literal(oracle):
    assert list(oracle.SLOT_FOR_K) == EXPECTED_SLOT_FOR_K
    assert list(ng.quant.SLOT_FOR_K) == EXPECTED_SLOT_FOR_K
    # the scalar decode formula of csrc/dequant.cuh:96
    assert [(4 + (k >> 1)) if (k & 1) else (k >> 1) for k in range(8)] == EXPECTED_SLOT_FOR_K


def test_known_answer_word(oracle):
    qu = np.arange(8, dtype=np.uint8).reshape(8, 1)
    word = int(oracle.pack_nibbles(qu).view(np.uint32)[0, 0])
    assert word == 0x75316420
    for k, slot in enumerate(EXPECTED_SLOT_FOR_K):
        assert (word >> (4 * slot)) & 0xF == k


def test_every_value_lands_in_its_slot(oracle):
    for k in range(8):
        for v in range(16):
            qu = np.zeros((8, 1), dtype=np.uint8)
            qu[k, 0] = v
            word = int(oracle.pack_nibbles(qu).view(np.uint32)[0, 0])
            assert word == v << (4 * EXPECTED_SLOT_FOR_K[k])


@pytest.mark.parametrize("shape", [(8, 1), (8, 4), (256, 64), (128, 130), (1024, 3), (2048, 1)])
def test_pack_unpack_involution_and_agreement(oracle, shape):
    K, N = shape
    qu = np.random.default_rng(K * 31 + N).integers(0, 16, size=shape, dtype=np.uint8)
    p_oracle = oracle.pack_nibbles(qu)
    p_pkg = ng.pack_nibbles(qu)
    assert p_pkg.dtype == np.int32 and p_pkg.shape == (K // 8, N)
    assert np.array_equal(p_oracle, p_pkg)
    assert np.array_equal(oracle.unpack_nibbles(p_oracle, K), qu)
    assert np.array_equal(ng.unpack_nibbles(p_pkg, K), qu)


def test_oracle_pack_rejections(oracle):
    with pytest.raises(ValueError):
        oracle.pack_nibbles(np.zeros((12, 4), dtype=np.uint8))
    bad = np.zeros((8, 4), dtype=np.uint8)
    bad[5, 2] = 16
    with pytest.raises(ValueError):
        oracle.pack_nibbles(bad)
    with pytest.raises(ValueError):
        oracle.unpack_nibbles(oracle.pack_nibbles(np.zeros((16, 4), np.uint8)), 24)


# --------------------------------------------------------------------------
# binary16
# --------------------------------------------------------------------------
def test_f16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_every_tie_and_neighbour(oracle):
    vals = np.unique(np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float64))
    vals = vals[np.isfinite(vals)]
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    extra = np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -25, 2.0 ** -26,
                      3 * 2.0 ** -26, 0.0, -0.0], dtype=np.float32)
    for arr in (mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                vals.astype(np.float32), extra):
        with np.errstate(over="ignore"):
            want = arr.astype(np.float16).view(np.uint16)
        assert np.array_equal(oracle.f32_to_f16(arr).view(np.uint16), want)


def test_f32_to_f16_random_bit_patterns(oracle):
    x = np.random.default_rng(7).integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64)
    x = x.astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x).view(np.uint16), want)


# --------------------------------------------------------------------------
# dequantize
# --------------------------------------------------------------------------
@pytest.mark.parametrize("group_size", [64, 128])
def test_dequant_unit_scales_is_n_minus_8(oracle, group_size):
    qu = sweep_nibbles(K=128)
    packed = oracle.pack_nibbles(qu)
    scales = np.ones((128 // group_size, qu.shape[1]), np.float16)
    W = oracle.dequantize(packed, scales, 128, group_size).astype(np.float32)
    assert np.array_equal(W, qu.astype(np.float32) - 8.0)
    assert W.min() == -8.0 and W.max() == 7.0


@pytest.mark.parametrize("group_size", [64, 128])
def test_dequant_power_of_two_scales_exact(oracle, group_size):
    qu = sweep_nibbles(K=256, seed=1)
    rows, N = 256 // group_size, qu.shape[1]
    e = np.random.default_rng(3).integers(-10, 11, size=(rows, N))
    scales = (2.0 ** e).astype(np.float16)
    W = oracle.dequantize(oracle.pack_nibbles(qu), scales, 256, group_size).astype(np.float64)
    want = (qu.astype(np.float64) - 8.0) * np.repeat(2.0 ** e, group_size, axis=0)
    assert np.array_equal(W, want)


@pytest.mark.parametrize("group_size", [64, 128])
def test_dequant_matches_numpy_single_rounding(oracle, group_size):
    qu = sweep_nibbles(K=256, seed=4)
    rows, N = 256 // group_size, qu.shape[1]
    rng = np.random.default_rng(5)
    scales = (2.0 ** rng.uniform(-14.0, 10.0, size=(rows, N))).astype(np.float16)
    W = oracle.dequantize(oracle.pack_nibbles(qu), scales, 256, group_size)
    # numpy: exact fp32 product of a small integer and an fp16 value, one RNE
    want = ((qu.astype(np.float32) - 8.0) *
            np.repeat(scales.astype(np.float32), group_size, axis=0)).astype(np.float16)
    assert np.array_equal(W.view(np.uint16), want.view(np.uint16))
    # and the package's host decode agrees bit for bit
    qw = ng.QuantizedWeight(torch.from_numpy(oracle.pack_nibbles(qu)),
                            torch.from_numpy(scales.copy()), group_size, 256, N)
    assert np.array_equal(ng.dequantize(qw).numpy().view(np.uint16), W.view(np.uint16))


@pytest.mark.parametrize("group_size", [64, 128])
def test_dequant_codebook_bound_and_group_index(oracle, group_size):
    qu = sweep_nibbles(K=512, extra_cols=4, seed=6)
    rows, N = 512 // group_size, qu.shape[1]
    # 2^row per group: reading a neighbouring group's scale is off by 2x
    scales = np.repeat((2.0 ** np.arange(rows))[:, None], N, axis=1).astype(np.float16)
    W = oracle.dequantize(oracle.pack_nibbles(qu), scales, 512, group_size).astype(np.float64)
    s = np.repeat(scales.astype(np.float64), group_size, axis=0)
    slack = 1.0 + 2.0 ** -11
    assert np.all(W <= 7.0 * s * slack) and np.all(W >= -8.0 * s * slack)
    assert np.array_equal(W, (qu - 8.0) * s)


# --------------------------------------------------------------------------
# RTN quantize
# --------------------------------------------------------------------------
def test_quantize_power_of_two_exact(oracle):
    rng = np.random.default_rng(8)
    K, N, g = 256, 24, 128
    e = rng.integers(-12, 4, size=(K // g, N))
    q = rng.integers(-7, 8, size=(K, N))
    q[::g] = 7  # max |q| = 7 in every group -> scale is exactly 2^e
    W = (q * np.repeat(2.0 ** e, g, axis=0)).astype(np.float32)
    qu, s32, s16 = oracle.quantize_rtn(W, g)
    assert np.array_equal(qu.astype(np.int64), q + 8)
    assert np.array_equal(s32, (2.0 ** e).astype(np.float32))
    assert np.array_equal(s16.astype(np.float64), 2.0 ** e)


def test_quantize_ties_round_half_even(oracle):
    g = 8
    base = np.array([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], dtype=np.float32)
    W = base.reshape(g, 1)
    qu, _, _ = oracle.quantize_rtn(W, g)
    assert (qu[:, 0].astype(int) - 8).tolist() == [7, 0, 2, 2, 0, -2, -2, 4]


def test_quantize_nearest_level_property(oracle):
    rng = np.random.default_rng(9)
    K, N, g = 512, 40, 128
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    qu, s32, s16 = oracle.quantize_rtn(W, g)
    s = np.repeat(s32.astype(np.float64), g, axis=0)
    q = qu.astype(np.float64) - 8.0
    # scale = max|w| / 7 per group and column
    amax = np.abs(W.reshape(K // g, g, N)).max(axis=1)
    assert np.array_equal(s32, np.maximum((amax / np.float32(7.0)).astype(np.float32), np.float32(1e-8)))
    # q is the nearest level to w / scale (within half a step, plus fp32 slack)
    assert np.all(np.abs(W / s - q) <= 0.5 + 1e-6)
    assert q.min() >= -8 and q.max() <= 7
    assert np.array_equal(s16, oracle.f32_to_f16(s32))


def test_quantize_zero_group(oracle):
    W = np.zeros((128, 3), np.float32)
    W[:, 1] = 1.0
    qu, s32, s16 = oracle.quantize_rtn(W, 128)
    assert np.all(qu[:, 0] == 8) and np.all(qu[:, 2] == 8)
    assert s32[0, 0] == np.float32(1e-8) and float(s16[0, 0]) == 0.0  # underflows in fp16
    assert np.all(qu[:, 1] == 15)


@pytest.mark.parametrize("g", [64, 128])
def test_package_quantize_matches_oracle(oracle, g):
    W = torch.randn(512, 72, generator=torch.Generator().manual_seed(g)) * 0.02
    qw = ng.quantize(W, group_size=g)
    qu, _, s16 = oracle.quantize_rtn(W.numpy(), g)
    assert np.array_equal(qw.qweight.numpy(), oracle.pack_nibbles(qu))
    assert np.array_equal(qw.scales.numpy().view(np.uint16), s16.view(np.uint16))


# --------------------------------------------------------------------------
# matmul
# --------------------------------------------------------------------------
def test_matmul_exact_on_integers(oracle):
    rng = np.random.default_rng(10)
    X = rng.integers(-8, 8, size=(5, 64)).astype(np.float16)
    W = rng.integers(-8, 8, size=(64, 36)).astype(np.float16)
    Y, Yf = oracle.matmul_f16w(X, W, want_f32=True)
    want = X.astype(np.int64) @ W.astype(np.int64)
    assert np.array_equal(Yf.astype(np.int64), want)
    assert np.array_equal(oracle.matmul_f64(X, W), want.astype(np.float64))
    # Y is X@W, not W^T@X^T or X@W^T: a transposed operand changes the shape
    assert Y.shape == (5, 36)


def test_matmul_f32_within_fp32_bound_of_f64(oracle):
    rng = np.random.default_rng(11)
    X = rng.standard_normal((4, 1024)).astype(np.float16)
    W = (rng.standard_normal((1024, 96)) * 0.05).astype(np.float16)
    _, Yf = oracle.matmul_f16w(X, W, want_f32=True)
    Yd = oracle.matmul_f64(X, W)
    bound = 1024 * 2.0 ** -24 * (np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)))
    assert np.all(np.abs(Yf - Yd) <= bound)
    assert np.allclose(Yd, X.astype(np.float64) @ W.astype(np.float64), rtol=0, atol=1e-9)


def test_reference_matmul_is_dequant_then_matmul(oracle):
    X, packed, scales = oracle.synthetic_case(3, 256, 64, 128, seed=3)
    Y = oracle.reference_matmul(X, packed, scales, 256, 128)
    W = oracle.dequantize(packed, scales, 256, 128)
    Yd = oracle.matmul_f64(X, W)
    assert oracle.rms_err(Y.astype(np.float64), Yd) < 1e-3
    # the package's torch reference_matmul agrees to fp32 summation order
    qw = ng.QuantizedWeight(torch.from_numpy(packed), torch.from_numpy(scales.copy()), 128, 256, 64)
    Yt = ng.reference_matmul(torch.from_numpy(X.copy()), qw).numpy()
    assert oracle.rms_err(Yt.astype(np.float64), Yd) < 1e-3


# --------------------------------------------------------------------------
# golden fixtures
# --------------------------------------------------------------------------
def test_golden_fixtures_regenerate(oracle):
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files})
    assert names, "no golden vectors"
    for name in names:
        if name.startswith("sweep"):
            K, N, g = z[f"{name}/meta"].tolist()
            W = oracle.dequantize(z[f"{name}/qweight"], z[f"{name}/scales"], K, g)
            assert np.array_equal(W.view(np.uint16), z[f"{name}/W"])
            continue
        M, K, N, g, seed = z[f"{name}/meta"].tolist()
        X, packed, scales = oracle.synthetic_case(M, K, N, g, seed)
        assert np.array_equal(X.view(np.uint16), z[f"{name}/X"])
        assert np.array_equal(packed, z[f"{name}/qweight"])
        assert np.array_equal(scales.view(np.uint16), z[f"{name}/scales"])
        W = oracle.dequantize(packed, scales, K, g)
        if f"{name}/W" in z.files:
            assert np.array_equal(W.view(np.uint16), z[f"{name}/W"])
        Y = oracle.matmul_f16w(X, W)
        assert np.array_equal(Y.view(np.uint16), z[f"{name}/Y"])


# --------------------------------------------------------------------------
# the package's device-resident quantiser and column concatenation (host run)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("g", [64, 128])
def test_quantize_device_matches_oracle_on_host(oracle, g):
    W = torch.randn(512, 72, generator=torch.Generator().manual_seed(g + 1)) * 0.02
    W[:g, 3] = 0.0  # an all-zero group: scale clamps to 1e-8
    qw = ng.quantize_device(W, group_size=g)
    qu, _, s16 = oracle.quantize_rtn(W.numpy(), g)
    assert np.array_equal(qw.qweight.numpy(), oracle.pack_nibbles(qu))
    assert np.array_equal(qw.scales.numpy().view(np.uint16), s16.view(np.uint16))


def test_concat_columns_is_the_packed_form_of_concatenated_weights(oracle):
    parts = [ng.quantize(torch.randn(256, n, generator=torch.Generator().manual_seed(n)) * 0.02, 128)
             for n in (64, 8, 132)]
    cat = ng.concat_columns(*parts)
    assert (cat.K, cat.N, cat.group_size) == (256, 204, 128)
    want = np.concatenate([oracle.dequantize(p.qweight.numpy(), p.scales.numpy(), 256, 128)
                           for p in parts], axis=1)
    got = oracle.dequantize(cat.qweight.numpy(), cat.scales.numpy(), 256, 128)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    with pytest.raises(ValueError):
        ng.concat_columns(parts[0], ng.quantize(torch.randn(128, 8), 128))
