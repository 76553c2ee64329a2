"""GPTQ / AWQ checkpoint ingestion (nibblegemm_amd.convert).

The checkpoint tensors are built here with plain numpy packers written from
the layout descriptions (sequential nibbles along K for GPTQ, zero points
stored as z - 1; column order [0, 2, 4, 6, 1, 3, 5, 7] along N for AWQ) and
checked two ways: the converted weight must pack to exactly what this
package's own packer gives for the same nibbles, and its dequantized values
must equal the checkpoint's ``(q - z) * s`` evaluated directly.
"""
import numpy as np
import pytest
import torch

from nibblegemm_amd import convert, quant
from nibblegemm_amd.quant import QuantizedWeight, dequantize, pack_nibbles

AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def _word(nibbles):
    """Eight 4-bit values -> int32 with value i in bits 4i..4i+3."""
    w = 0
    for i, v in enumerate(nibbles):
        w |= (int(v) & 0xF) << (4 * i)
    return np.array(w, dtype=np.uint32).view(np.int32)


def gptq_pack(n, z, g, zero_offset=1):
    K, N = n.shape
    qweight = np.empty((K // 8, N), dtype=np.int32)
    for r in range(K // 8):
        for c in range(N):
            qweight[r, c] = _word(n[8 * r:8 * r + 8, c])
    qzeros = np.empty((K // g, N // 8), dtype=np.int32)
    for gi in range(K // g):
        for c in range(N // 8):
            qzeros[gi, c] = _word(z[gi, 8 * c:8 * c + 8] - zero_offset)
    return torch.from_numpy(qweight), torch.from_numpy(qzeros)


def awq_pack(n):
    R, N = n.shape
    out = np.empty((R, N // 8), dtype=np.int32)
    for r in range(R):
        for c in range(N // 8):
            out[r, c] = _word([n[r, 8 * c + AWQ_ORDER[i]] for i in range(8)])
    return torch.from_numpy(out)


def _case(K=256, N=64, g=64, seed=0):
    rng = np.random.default_rng(seed)
    n = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    scales = torch.from_numpy(rng.uniform(0.002, 0.02, size=(K // g, N)).astype(np.float16))
    return n, scales


def _direct_dequant(n, z, scales, g):
    """(q - z) * s in fp32, rounded once to fp16: the checkpoints' own definition."""
    s = scales.float().repeat_interleave(g, dim=0)
    zz = torch.from_numpy(np.repeat(z, g, axis=0).astype(np.float32))
    return ((torch.from_numpy(n.astype(np.float32)) - zz) * s).to(torch.float16)


@pytest.mark.parametrize("zero_offset", [1, 0])
def test_gptq_symmetric_converts_exactly(zero_offset):
    K, N, g = 256, 64, 64
    n, scales = _case(K, N, g)
    z = np.full((K // g, N), 8, dtype=np.int64)
    qweight, qzeros = gptq_pack(n, z, g, zero_offset)
    qw = convert.from_gptq(qweight, qzeros, scales, g, zero_offset=zero_offset)
    assert (qw.K, qw.N, qw.group_size) == (K, N, g)
    assert np.array_equal(qw.qweight.numpy(), pack_nibbles(n))
    assert torch.equal(qw.scales, scales)
    assert torch.equal(dequantize(qw), _direct_dequant(n, z, scales, g))


def test_gptq_trivial_g_idx_accepted_act_order_rejected():
    K, N, g = 256, 64, 128
    n, scales = _case(K, N, g, seed=1)
    qweight, qzeros = gptq_pack(n, np.full((K // g, N), 8), g)
    ok = torch.arange(K, dtype=torch.int32) // g
    qw = convert.from_gptq(qweight, qzeros, scales, g, g_idx=ok)
    assert np.array_equal(qw.qweight.numpy(), pack_nibbles(n))
    perm = ok[torch.randperm(K, generator=torch.Generator().manual_seed(0))]
    with pytest.raises(ValueError, match="act-order"):
        convert.from_gptq(qweight, qzeros, scales, g, g_idx=perm)


def test_gptq_asymmetric_rejected():
    K, N, g = 128, 16, 64
    n, scales = _case(K, N, g, seed=2)
    z = np.full((K // g, N), 8)
    z[1, 5] = 3
    qweight, qzeros = gptq_pack(n, z, g)
    with pytest.raises(ValueError, match="zero points other than 8"):
        convert.from_gptq(qweight, qzeros, scales, g)


def test_gptq_shape_errors():
    K, N, g = 128, 16, 64
    n, scales = _case(K, N, g, seed=3)
    qweight, qzeros = gptq_pack(n, np.full((K // g, N), 8), g)
    with pytest.raises(ValueError, match="scales"):
        convert.from_gptq(qweight, qzeros, scales[:1], g)
    with pytest.raises(ValueError, match="qzeros"):
        convert.from_gptq(qweight, qzeros[:, :1], scales, g)
    with pytest.raises(ValueError, match="int32"):
        convert.from_gptq(qweight.to(torch.int64), qzeros, scales, g)


@pytest.mark.parametrize("zero_offset", [1, 0])
def test_to_gptq_round_trip(zero_offset):
    K, N, g = 256, 32, 128
    n, scales = _case(K, N, g, seed=4)
    qw = QuantizedWeight(torch.from_numpy(pack_nibbles(n)), scales, g, K, N)
    qweight, qzeros, s, g_idx = convert.to_gptq(qw, zero_offset=zero_offset)
    # the exported tensors are exactly what the reference packer of the layout gives
    eq, ez = gptq_pack(n, np.full((K // g, N), 8), g, zero_offset)
    assert torch.equal(qweight, eq) and torch.equal(qzeros, ez)
    assert torch.equal(s, scales)
    assert torch.equal(g_idx, torch.arange(K, dtype=torch.int32) // g)
    back = convert.from_gptq(qweight, qzeros, s, g, g_idx=g_idx, zero_offset=zero_offset)
    assert torch.equal(back.qweight, qw.qweight) and torch.equal(back.scales, qw.scales)


def test_awq_symmetric_converts_exactly():
    K, N, g = 256, 64, 64
    n, scales = _case(K, N, g, seed=5)
    z = np.full((K // g, N), 8, dtype=np.int64)
    qw = convert.from_awq(awq_pack(n), awq_pack(z), scales, g)
    assert (qw.K, qw.N) == (K, N)
    assert np.array_equal(qw.qweight.numpy(), pack_nibbles(n))
    assert torch.equal(dequantize(qw), _direct_dequant(n, z, scales, g))


def test_awq_asymmetric_rejected():
    K, N, g = 128, 16, 64
    n, scales = _case(K, N, g, seed=6)
    z = np.full((K // g, N), 8)
    z[0, 9] = 12
    with pytest.raises(ValueError, match="zero points other than 8"):
        convert.from_awq(awq_pack(n), awq_pack(z), scales, g)


def test_pack_interleaved_matches_host_packer():
    rng = np.random.default_rng(7)
    n = rng.integers(0, 16, size=(64, 40), dtype=np.uint8)
    got = convert.pack_interleaved(torch.from_numpy(n.astype(np.int64)))
    assert np.array_equal(got.numpy(), pack_nibbles(n))
    assert got.dtype == torch.int32


def test_top_slot_sign_bit():
    # k = 7 lives in slot 7 (bits 28..31): a value >= 8 there sets the int32 sign bit.
    n = np.zeros((8, 1), dtype=np.uint8)
    n[7, 0] = 15
    got = convert.pack_interleaved(torch.from_numpy(n.astype(np.int64)))
    assert int(got[0, 0]) == np.array(0xF0000000, dtype=np.uint32).view(np.int32)
    assert quant.SLOT_FOR_K[7] == 7


@pytest.mark.gpu
def test_convert_on_device_matches_host():
    K, N, g = 512, 128, 128
    n, scales = _case(K, N, g, seed=8)
    qweight, qzeros = gptq_pack(n, np.full((K // g, N), 8), g)
    host = convert.from_gptq(qweight, qzeros, scales, g)
    dev = convert.from_gptq(qweight.cuda(), qzeros.cuda(), scales.cuda(), g)
    assert dev.qweight.is_cuda
    assert torch.equal(dev.qweight.cpu(), host.qweight)
    assert torch.equal(dev.scales.cpu(), host.scales)
