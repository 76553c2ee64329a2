"""The packed nibble format, on the host: the layout every kernel decodes.

CPU only.  The slot table and the word 0x75316420 are the reference's
known-answer data (tests/test_pack.py:17, :42 there); the checks around them
are this package's: every (slot, code) bit position, agreement with the C
oracle's independent packer, both round trips, and the input validation of
the drop-in functions (ValueError, as in python/nibblegemm/quant.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import quant
from nibblegemm_amd.quant import PACK_FACTOR, SLOT_FOR_K, dequantize, quantize

SLOT_TABLE = (0, 4, 1, 5, 2, 6, 3, 7)  # known-answer data: slot of k = 0..7
ASCENDING_WORD = 0x75316420  # known-answer data: codes k = 0..7 packed


def test_format_constants():
    assert tuple(SLOT_FOR_K) == SLOT_TABLE
    assert (quant.QMIN, quant.QMAX, quant.ZERO_POINT, quant.PACK_FACTOR) == (-8, 7, 8, 8)
    # K_FOR_SLOT inverts the table; even k live in slots 0..3, odd k in 4..7.
    assert [int(quant.K_FOR_SLOT[SLOT_FOR_K[k]]) for k in range(8)] == list(range(8))
    assert [SLOT_TABLE[k] // 4 for k in range(8)] == [k % 2 for k in range(8)]


def test_every_code_lands_in_its_slot():
    """A column holding one nonzero code c at offset k packs to exactly
    c << (4 * slot(k)): all 8 offsets x 15 codes."""
    for k in range(8):
        qu = np.zeros((8, 15), np.uint8)
        qu[k, :] = np.arange(1, 16)
        words = ng.pack_nibbles(qu).view(np.uint32)[0]
        assert words.tolist() == [c << (4 * SLOT_TABLE[k]) for c in range(1, 16)]


def test_ascending_codes_known_answer():
    qu = np.arange(8, dtype=np.uint8)[:, None]
    assert int(ng.pack_nibbles(qu).view(np.uint32)[0, 0]) == ASCENDING_WORD
    # and read back, slot by slot
    assert [(ASCENDING_WORD >> (4 * s)) & 0xF for s in SLOT_TABLE] == list(range(8))


@pytest.mark.parametrize("K,N,seed", [(8, 5, 0), (64, 33, 1), (512, 96, 2), (4096, 7, 3)])
def test_packer_agrees_with_the_oracle_and_round_trips(oracle, K, N, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    packed = ng.pack_nibbles(codes)
    assert packed.dtype == np.int32 and packed.shape == (K // 8, N)
    assert np.array_equal(packed, oracle.pack_nibbles(codes))
    assert np.array_equal(ng.unpack_nibbles(packed, K), codes)
    # arbitrary words (negative int32 included) survive unpack -> pack
    words = rng.integers(-(1 << 31), 1 << 31, size=(K // 8, N), dtype=np.int64).astype(np.int32)
    assert np.array_equal(ng.pack_nibbles(ng.unpack_nibbles(words, K)), words)


def test_high_codes_at_k7_make_negative_words():
    qu = np.zeros((8, 16), np.uint8)
    qu[7, :] = np.arange(16)  # k = 7 sits in the top nibble
    words = ng.pack_nibbles(qu)[0].astype(np.int64)
    assert ((words < 0) == (np.arange(16) >= 8)).all()
    assert words[15] == -(1 << 31) + (7 << 28)


def test_negative_signed_codes_wrap_into_their_own_nibble():
    """A signed input passes the > 15 check with negative codes; each one is
    masked to its low four bits before the shift (the reference's ``& 0xF``,
    python/nibblegemm/quant.py:177), so -c packs as 16 - c in its own slot and
    leaves every other nibble of the word untouched."""
    for k in range(8):
        qu = np.zeros((8, 8), np.int8)
        qu[k, :] = -np.arange(1, 9, dtype=np.int8)
        words = ng.pack_nibbles(qu).view(np.uint32)[0]
        assert words.tolist() == [(16 - c) << (4 * SLOT_TABLE[k]) for c in range(1, 9)]
    rng = np.random.default_rng(5)
    codes = rng.integers(-8, 8, size=(64, 9)).astype(np.int8)
    assert np.array_equal(ng.pack_nibbles(codes), ng.pack_nibbles((codes & 0xF).astype(np.uint8)))


def _bad_pack_value():
    qu = np.zeros((16, 3), np.uint8)
    qu[9, 1] = 200
    return lambda: ng.pack_nibbles(qu)


@pytest.mark.parametrize("call,needle", [
    (lambda: ng.pack_nibbles(np.zeros((20, 2), np.uint8)), "divisible by 8"),
    (_bad_pack_value(), "4 bits"),
    (lambda: ng.unpack_nibbles(np.zeros((3, 2), np.int32), 32), "inconsistent"),
    (lambda: quantize(torch.zeros(2, 3, 128)), "2-D"),
    (lambda: quantize(torch.zeros(320, 4), group_size=128), "divisible by group_size"),
    (lambda: quantize(torch.zeros(96, 4), group_size=12), "divisible by 8"),
    (lambda: ng.quantize_device(torch.zeros(200, 4), group_size=64), "divisible by group_size"),
])
def test_invalid_inputs_raise_value_error(call, needle):
    with pytest.raises(ValueError, match=needle):
        call()


def test_quantized_weight_accounting_and_move():
    qw = quantize(torch.randn(384, 20) * 0.02, group_size=64)
    assert qw.qweight.dtype == torch.int32 and tuple(qw.qweight.shape) == (48, 20)
    assert qw.scales.dtype == torch.float16 and tuple(qw.scales.shape) == (6, 20)
    assert qw.weight_bytes == 48 * 20 * 4 + 6 * 20 * 2
    moved = qw.to("cpu")
    assert (moved.K, moved.N, moved.group_size) == (384, 20, 64)
    assert torch.equal(moved.qweight, qw.qweight) and torch.equal(moved.scales, qw.scales)


def test_interleave_swiglu_column_order():
    """Columns alternate gate/up in blocks of 16; split_swiglu inverts it."""
    from nibblegemm_amd.quant import QuantizedWeight, interleave_swiglu, split_swiglu
    K, N, g = 16, 64, 8
    gq = torch.arange(K // 8 * N, dtype=torch.int32).reshape(K // 8, N)
    uq = -1 - gq
    gs = torch.arange(K // g * N, dtype=torch.float32).reshape(K // g, N).half()
    us = -gs
    qw = interleave_swiglu(QuantizedWeight(gq, gs, g, K, N), QuantizedWeight(uq, us, g, K, N))
    assert (qw.K, qw.N) == (K, 2 * N)
    for b in range(N // 16):
        assert torch.equal(qw.qweight[:, 32 * b:32 * b + 16], gq[:, 16 * b:16 * b + 16])
        assert torch.equal(qw.qweight[:, 32 * b + 16:32 * b + 32], uq[:, 16 * b:16 * b + 16])
        assert torch.equal(qw.scales[:, 32 * b + 16:32 * b + 32], us[:, 16 * b:16 * b + 16])
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
