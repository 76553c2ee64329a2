"""On-disk nibble format of the package (reference tests/test_pack.py intents).

CPU only: pins the layout every kernel decodes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import quant
from nibblegemm_amd.quant import PACK_FACTOR, SLOT_FOR_K, dequantize, quantize

EXPECTED_SLOT_FOR_K = [0, 4, 1, 5, 2, 6, 3, 7]


def test_slot_table_is_the_documented_permutation():
    assert list(SLOT_FOR_K) == EXPECTED_SLOT_FOR_K
    assert list(ng.quant.K_FOR_SLOT) == [0, 2, 4, 6, 1, 3, 5, 7]


def test_slot_table_matches_the_cuda_scalar_decode():
    """The reference's scalar decode computes the slot instead of looking it
    up (csrc/dequant.cuh:96: odd k in the high half of the word); the formula
    gives the documented table."""
    slot = [(4 + (k >> 1)) if (k & 1) else (k >> 1) for k in range(PACK_FACTOR)]
    assert slot == EXPECTED_SLOT_FOR_K


def test_nibble_slot_assignment_is_pinned():
    qu = np.arange(PACK_FACTOR, dtype=np.uint8).reshape(PACK_FACTOR, 1)
    word = int(ng.pack_nibbles(qu).view(np.uint32)[0, 0])
    for k, slot in enumerate(EXPECTED_SLOT_FOR_K):
        assert (word >> (4 * slot)) & 0xF == k
    assert word == 0x75316420


@pytest.mark.parametrize("shape", [(8, 1), (8, 4), (256, 64), (128, 130), (1024, 3), (2048, 1)])
def test_pack_unpack_is_an_involution(shape):
    K, N = shape
    qu = np.random.default_rng(K * 31 + N).integers(0, 16, size=shape, dtype=np.uint8)
    packed = ng.pack_nibbles(qu)
    assert packed.dtype == np.int32
    assert packed.shape == (K // PACK_FACTOR, N)
    assert np.array_equal(ng.unpack_nibbles(packed, K), qu)


def test_top_nibble_sets_the_sign_bit():
    qu = np.zeros((8, 1), np.uint8)
    qu[7, 0] = 15  # k = 7 lives in slot 7, bits 28..31
    assert int(ng.pack_nibbles(qu)[0, 0]) == -(1 << 31) + (7 << 28)


def test_pack_rejects_values_above_15():
    qu = np.zeros((8, 4), dtype=np.uint8)
    qu[5, 2] = 16
    with pytest.raises(ValueError):
        ng.pack_nibbles(qu)


def test_pack_rejects_k_not_divisible_by_8():
    with pytest.raises(ValueError):
        ng.pack_nibbles(np.zeros((12, 4), dtype=np.uint8))


def test_unpack_rejects_inconsistent_k():
    packed = ng.pack_nibbles(np.zeros((16, 4), dtype=np.uint8))
    with pytest.raises(ValueError):
        ng.unpack_nibbles(packed, 24)


@pytest.mark.parametrize("K,group_size", [(192, 128), (100, 64), (8, 128), (130, 128)])
def test_quantize_rejects_k_not_divisible_by_group(K, group_size):
    with pytest.raises(ValueError):
        ng.quantize(torch.randn(K, 8), group_size=group_size)


def test_quantize_rejects_non_2d_weight():
    with pytest.raises(ValueError):
        ng.quantize(torch.randn(4, 128, 8), group_size=128)


def test_quantize_rejects_group_not_multiple_of_8():
    with pytest.raises(ValueError):
        ng.quantize(torch.randn(120, 8), group_size=12)


def test_quantized_weight_bytes_and_to():
    qw = ng.quantize(torch.randn(256, 16) * 0.02, group_size=128)
    assert qw.qweight.shape == (32, 16) and qw.qweight.dtype == torch.int32
    assert qw.scales.shape == (2, 16) and qw.scales.dtype == torch.float16
    assert qw.weight_bytes == 32 * 16 * 4 + 2 * 16 * 2
    qw2 = qw.to("cpu")
    assert torch.equal(qw2.qweight, qw.qweight) and (qw2.K, qw2.N, qw2.group_size) == (256, 16, 128)


def test_interleave_swiglu_column_order():
    """Columns alternate gate/up in blocks of 32; split_swiglu inverts it."""
    import torch
    from nibblegemm_amd.quant import QuantizedWeight, interleave_swiglu, split_swiglu
    K, N, g = 16, 64, 8
    gq = torch.arange(K // 8 * N, dtype=torch.int32).reshape(K // 8, N)
    uq = -1 - gq
    gs = torch.arange(K // g * N, dtype=torch.float32).reshape(K // g, N).half()
    us = -gs
    qw = interleave_swiglu(QuantizedWeight(gq, gs, g, K, N), QuantizedWeight(uq, us, g, K, N))
    assert (qw.K, qw.N) == (K, 2 * N)
    assert torch.equal(qw.qweight[:, :32], gq[:, :32]) and torch.equal(qw.qweight[:, 32:64], uq[:, :32])
    assert torch.equal(qw.qweight[:, 64:96], gq[:, 32:]) and torch.equal(qw.scales[:, 96:], us[:, 32:])
    g_back, u_back = split_swiglu(qw.qweight)
    assert torch.equal(g_back, gq) and torch.equal(u_back, uq)


# ---------------------------------------------------------------------------
# quantize(clip_search=True): the reference's MSE scale search (quant.py:81-124)
# ---------------------------------------------------------------------------
def _clip_case(K=256, N=96, seed=0):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(K, N, generator=g) * 0.02
    W[torch.rand(K, N, generator=g) < 0.01] *= 8  # outliers: clipping pays for some groups
    return W


def _group_sse(W, scales, G):
    """Squared quantisation error per (group, column) in float64."""
    K, N = W.shape
    g = W.double().reshape(K // G, G, N)
    s = scales.double().unsqueeze(1)
    q = torch.round(g / s).clamp(-8, 7)
    return (q * s - g).pow(2).sum(dim=1)


def test_clip_search_scale_is_a_candidate_and_never_worse():
    """The chosen scale is one of the 19 clipped max-abs scales, and its
    squared error is no larger than max-abs's (ratio 1 is the first candidate
    and is replaced only by a strictly better one)."""
    W, G = _clip_case(), 128
    groups = W.float().reshape(-1, G, W.shape[1])
    chosen = quant._search_scale(groups)
    amax = groups.abs().amax(dim=1)
    cands = torch.stack([(amax * r / 7).clamp(min=1e-8) for r in quant.CLIP_RATIOS])
    assert bool((cands == chosen.unsqueeze(0)).any(dim=0).all())
    plain = (amax / 7).clamp(min=1e-8)
    assert bool((_group_sse(W, chosen, G) <= _group_sse(W, plain, G) * (1 + 1e-6)).all())
    assert bool((chosen < plain).any())  # the outliers make clipping win somewhere


def test_clip_search_picks_the_minimum_error_ratio():
    """Brute force in float64 over the same candidates agrees with the search
    (float32 sums may order near-equal candidates differently: allow a few)."""
    W, G = _clip_case(seed=1), 64
    groups = W.float().reshape(-1, G, W.shape[1])
    chosen = quant._search_scale(groups)
    amax = groups.abs().amax(dim=1)
    cands = torch.stack([(amax * r / 7).clamp(min=1e-8) for r in quant.CLIP_RATIOS])
    sse = torch.stack([_group_sse(W, c, G) for c in cands])
    best = cands.gather(0, sse.argmin(dim=0, keepdim=True))[0]
    assert (best != chosen).float().mean().item() < 0.02


def test_quantize_with_clip_search_uses_the_searched_scales():
    W, G = _clip_case(seed=2), 128
    qw = quantize(W, G, clip_search=True)
    scales = quant._search_scale(W.float().reshape(-1, G, W.shape[1]))
    assert torch.equal(qw.scales, scales.half())
    deq = dequantize(qw).float()
    rtn = dequantize(quantize(W, G)).float()
    assert (deq - W).pow(2).mean() < (rtn - W).pow(2).mean()
