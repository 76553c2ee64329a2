"""Seeded random shapes through every kernel entry point, against the oracle.

The fixed-shape tests pin the edge cases the reference's own tests name;
this sweep covers what falls between them: M, K and N drawn at random (N a
multiple of 2 or 4 as each entry point requires, K a multiple of the group
size), so tile tails, strip tails, row blocks and K splits meet in
combinations no hand-picked case lists.  Shapes stay small enough for the
C oracle to finish in well under a second each.

Bounds as in the fixed tests: bit-exact for dequant; ``max|y - ref| <=
1e-2 * rms(ref)`` and the reference's ``max|y - ref| / mean|ref| < 3e-2``
for the matmuls.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
import oracle
from cases import host, oracle_y, rel_err, rms_err, synthetic

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-2
REL_TOL = 3e-2


def _shapes(seed: int, n: int, m_max: int, n_mult: int):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        g = rng.choice([64, 128])
        K = g * rng.randint(1, 24)
        N = n_mult * rng.randint(1, 700 // n_mult)
        M = rng.randint(1, m_max)
        out.append((M, K, N, g))
    return out


@pytest.mark.parametrize("M,K,N,g", _shapes(101, 24, 8, 4))
def test_gemv_random_shapes(M, K, N, g):
    X, packed, scales, Xd, qw = synthetic(M, K, N, g, seed=M * 7 + K + N)
    ref = oracle_y(X, packed, scales, K, g)
    for version in (2, 3, 4):
        y = host(ng.gemv(Xd, qw, version=version))
        assert rms_err(y, ref) <= RMS_TOL, (version, rms_err(y, ref))
        assert rel_err(y, ref) < REL_TOL
    assert torch.equal(ng.gemv(Xd, qw, version=3), ng.gemv(Xd, qw, version=4, splits=1))


@pytest.mark.parametrize("M,K,N,g", _shapes(202, 24, 300, 2) + _shapes(203, 6, 1300, 4))
def test_gemm_random_shapes(M, K, N, g):
    X, packed, scales, Xd, qw = synthetic(M, K, N, g, seed=M * 7 + K + N)
    ref = oracle_y(X, packed, scales, K, g)
    for version in (6, 7):
        y = host(ng.gemm(Xd, qw, version=version))
        assert rms_err(y, ref) <= RMS_TOL, (version, rms_err(y, ref))
        assert rel_err(y, ref) < REL_TOL
    assert torch.equal(ng.matmul(Xd, qw), ng.gemv(Xd, qw) if M <= ng.DECODE_MAX_M else ng.gemm(Xd, qw))


@pytest.mark.parametrize("M,K,N,g", _shapes(303, 12, 128, 4))
def test_bias_epilogue_random_shapes(M, K, N, g):
    """The fused bias epilogue is the product then an fp16 add, to the bit."""
    _, _, _, Xd, qw = synthetic(M, K, N, g, seed=M + K * 3 + N)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(N)).half().to("cuda")
    assert torch.equal(ng.ops.matmul_bias(Xd, qw, bias), ng.matmul(Xd, qw) + bias)


@pytest.mark.parametrize("K,N,g", [s[1:] for s in _shapes(404, 16, 1, 2)])
def test_dequant_random_shapes(K, N, g):
    rng = np.random.default_rng(K * 31 + N)
    qu = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    scales = rng.uniform(0.002, 0.02, size=(K // g, N)).astype(np.float16)
    packed = ng.pack_nibbles(qu)
    qw = ng.QuantizedWeight(torch.from_numpy(packed), torch.from_numpy(scales), g, K, N).to("cuda")
    expect = oracle.dequantize(packed, scales, K, g)
    for fast in (True, False):
        got = ng.dequant(qw, fast=fast).cpu().numpy()
        assert got.dtype == np.float16 and np.array_equal(got.view(np.uint16), expect.view(np.uint16))


def _glue_cases(seed: int, n: int):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        n_kv = rng.choice([1, 2, 8])
        n_heads = n_kv * rng.choice([1, 2, 4, 8])
        max_seq = rng.randint(1, 3000)
        out.append((n_heads, n_kv, rng.randrange(max_seq), max_seq))
    return out


@pytest.mark.parametrize("n_heads,n_kv,pos,max_seq", _glue_cases(505, 16))
def test_attention_random_positions(n_heads, n_kv, pos, max_seq):
    """Grouped-query attention at random positions, head ratios and cache
    sizes (one chunk to two dozen), against the float32 reference, to one
    fp16 rounding of the output; a repeat gives the same bits."""
    from test_glue import _attn_case, err_rms, ref_attention, ulp_excess

    from nibblegemm_amd import glue

    qkv, kc, vc = _attn_case(n_heads, n_kv, pos, max_seq, seed=pos + 17 * n_heads + max_seq)
    rope = glue.rope_tables(max_seq)
    ref, _, _ = ref_attention(qkv, kc, vc, pos, n_heads, n_kv, rope)
    a = glue.attention_decode(qkv, kc, vc, pos, rope)
    assert err_rms(a, ref) <= 1e-2
    assert ulp_excess(a, ref) <= 1.0, ulp_excess(a, ref)
    assert torch.equal(glue.attention_decode(qkv, kc, vc, pos, rope), a)


@pytest.mark.parametrize("M,K,N,g", [(m % 8 + 1, k, n, g) for m, k, n, g in _shapes(606, 16, 8, 4)])
def test_rmsnorm_matmul_random_shapes(M, K, N, g):
    """The RMSNorm prologue gives the bits of the RMSNorm launch followed by
    the matmul, at random shapes (K a multiple of 8 up to 16384 columns)."""
    from nibblegemm_amd import glue, ops

    gen = torch.Generator().manual_seed(M + K + N)
    qw = ng.quantize(torch.randn((K, N), generator=gen) * 0.02, g).to("cuda")
    x = (torch.randn((M, K), generator=gen) * 2).half().to("cuda")
    w = (1 + 0.1 * torch.randn(K, generator=gen)).half().to("cuda")
    assert torch.equal(ops.rmsnorm_matmul(x, w, qw, 1e-5), ops.matmul(glue.rmsnorm(x, w, 1e-5), qw))
