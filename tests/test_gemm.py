"""Parity of the MFMA prefill GEMM with the reference path.

Edge cases follow the reference's tests/test_gemm.py (M on, just past and far
past tile boundaries; N with masked columns), then the benchmark prefill and
handover configs at full size: sampled rows against the CPU oracle at every
prefill point, every output against it at the bench's M = 2048 points (the
C oracle takes a few seconds there on the host's cores).

Bounds: north-star ``max|y - ref| <= 1e-2 * rms(ref)`` and the reference's
``max|y - ref| / mean|ref| < 3e-2`` (tests/test_gemm.py:34 there).  The LDS B
tile holds exactly the oracle's dequantized fp16 values and MFMA accumulates
in fp32, so only summation order and the final fp16 rounding differ.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import quant
from cases import host, oracle_y, oracle_y_rows, quantized, rel_err, rms_err, synthetic, to_dev_qw

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-2
REL_TOL = 3e-2
K = 256
M_VALUES = [1, 17, 64, 65, 128, 1000]
N_VALUES = [128, 132]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w4a16_golden.npz")


@pytest.mark.parametrize("version", [6, 7])
@pytest.mark.parametrize("M", M_VALUES)
@pytest.mark.parametrize("N", N_VALUES)
@pytest.mark.parametrize("group_size", [64, 128])
def test_gemm_matches_reference(version, M, N, group_size):
    X, packed, scales, Xd, qw = quantized(M, K, N, group_size)
    y = ng.gemm(Xd, qw, version=version)
    assert y.shape == (M, N) and y.dtype == torch.float16
    ref = oracle_y(X, packed, scales, K, group_size)
    assert rms_err(host(y), ref) <= RMS_TOL
    assert rel_err(host(y), ref) < REL_TOL


@pytest.mark.parametrize("M", [16, 64, 512])
def test_matmul_dispatches_to_gemm_above_the_crossover(M):
    _, _, _, Xd, qw = quantized(M, K, 128, 128, seed=1)
    assert M > ng.DECODE_MAX_M
    assert torch.equal(ng.matmul(Xd, qw), ng.gemm(Xd, qw))


@pytest.mark.parametrize("M", [9, 33, 200])
@pytest.mark.parametrize("K_,N", [(512, 130), (1024, 4102), (192, 64)])
def test_gemm_odd_shapes(M, K_, N):
    g = 64 if K_ % 128 else 128
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M + N)
    ref = oracle_y(X, packed, scales, K_, g)
    for version in (6, 7):
        assert rms_err(host(ng.gemm(Xd, qw, version=version)), ref) <= RMS_TOL


def test_versions_agree():
    _, _, _, Xd, qw = synthetic(300, 1024, 640, 128, seed=3)
    a, b = host(ng.gemm(Xd, qw, version=6)), host(ng.gemm(Xd, qw, version=7))
    assert rel_err(a, b) < REL_TOL


@pytest.mark.parametrize("M", [16, 32])
def test_small_batch_config_gemm_leg(M):
    """The small-batch config (M = 16, 32 at 4096 x 14336) above M = 8, the GEMM side
    of the handover, at full size."""
    X, packed, scales, Xd, qw = synthetic(M, 4096, 14336, 128, seed=200 + M)
    y = host(ng.matmul(Xd, qw))
    assert rms_err(y, oracle_y(X, packed, scales, 4096, 128)) <= RMS_TOL


@pytest.mark.parametrize("M", [12, 16, 17, 24, 32])
@pytest.mark.parametrize("K_,N", [(4096, 14336), (14336, 4096)])
def test_batch_rows_full_size(M, K_, N):
    """12..32 rows at the small-batch config's full sizes (the batch kernel:
    each step's activation window copied into an LDS ring by staging waves;
    12 and 16 rows at 4096 x 14336 take the 16-row strip kernel), every
    output against the oracle; repeated calls bit-identical."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=700 + M + K_)
    y = ng.gemm(Xd, qw)
    assert torch.equal(ng.gemm(Xd, qw), y)
    ref = oracle_y(X, packed, scales, K_, 128)
    assert rms_err(host(y), ref) <= RMS_TOL
    assert rel_err(host(y), ref) < REL_TOL


@pytest.mark.parametrize("M,K_,N", [(M, K_, N) for M in (33, 48, 64)
                                    for K_, N in ((4096, 14336), (14336, 4096), (8192, 8192))]
                         + [(40, 4096, 4096), (57, 14336, 4036)])
def test_batch_64_row_block(M, K_, N):
    """33..64 rows whose one 64-row block makes one round of the CUs run the
    batch kernel in that block: every output against an fp32 product of the
    dequant kernel's weights, both versions and matmul the same bits,
    repeated calls bit-identical.  The last shape ends in a partial strip."""
    ext = ng.extension()
    assert ext.gemm_streams(M, K_, N, 128)
    _, _, _, Xd, qw = synthetic(M, K_, N, 128, seed=800 + M + N)
    ref = Xd.float() @ ng.dequant(qw).float()
    rms = ref.pow(2).mean().sqrt()
    y = ng.gemm(Xd, qw, version=6)
    assert torch.equal(ng.gemm(Xd, qw, version=7), y)
    assert torch.equal(ng.gemm(Xd, qw), y)
    assert torch.equal(ng.matmul(Xd, qw), y)
    assert torch.isfinite(y.float()).all()
    assert float((y.float() - ref).abs().max() / rms) <= RMS_TOL


@pytest.mark.parametrize("M", [33, 64])
def test_batch_64_row_block_against_the_oracle(M):
    """The small-batch config's down projection (14336 x 4096) at 33 and 64
    rows, every output against the CPU oracle."""
    X, packed, scales, Xd, qw = synthetic(M, 14336, 4096, 128, seed=850 + M)
    y = host(ng.gemm(Xd, qw))
    ref = oracle_y(X, packed, scales, 14336, 128)
    assert rms_err(y, ref) <= RMS_TOL
    assert rel_err(y, ref) < REL_TOL


@pytest.mark.parametrize("M,K_,N", [(17, 4096, 28672), (32, 4096, 28672), (24, 4096, 30720),
                                    (20, 4096, 28736), (24, 4096, 32768)])
def test_batch_strip_pairs(M, K_, N):
    """Where pairs of adjacent strips make one round of the CUs without a K
    split (448..512 strips), a workgroup takes a pair and copies the
    activation window once for both.  Each output keeps its arithmetic: the
    result has the bits of the two column halves computed apart (a cut
    mid-strip included), matches the oracle (the fused gate|up shape) or an
    fp32 product of the dequant kernel's weights, repeats its bits, and
    replays from a graph.  28736 columns end in an unpaired strip."""
    ext = ng.extension()
    assert ext.gemm_workspace_bytes(M, K_, N, 128, 6, None) == (0, 0)  # no K split
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=900 + M + N)
    y = ng.gemm(Xd, qw)
    assert torch.equal(ng.gemm(Xd, qw), y)
    half = N // 2
    parts = [ng.gemm(Xd, quant.QuantizedWeight(qw.qweight[:, a:b].contiguous(),
                                               qw.scales[:, a:b].contiguous(), 128, K_, b - a))
             for a, b in ((0, half), (half, N))]
    assert torch.equal(torch.cat(parts, dim=1), y)
    if N == 28672:
        ref = oracle_y(X, packed, scales, K_, 128)
        assert rms_err(host(y), ref) <= RMS_TOL
        assert rel_err(host(y), ref) < REL_TOL
    else:
        ref = Xd.float() @ ng.dequant(qw).float()
        assert float((y.float() - ref).abs().max() / ref.pow(2).mean().sqrt()) <= RMS_TOL
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ng.gemm(Xd, qw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        out = ng.gemm(Xd, qw)
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)


@pytest.mark.parametrize("M,K_,N,g", [(24, 14336, 4096, 128), (17, 4096, 1024, 128), (32, 2048, 1540, 64),
                                      (20, 640, 196, 64), (14, 14336, 1024, 128), (12, 1024, 260, 64),
                                      (48, 14336, 4096, 128)])
def test_batch_rows_replay_in_a_graph(M, K_, N, g):
    """The batch kernel with K split (4, 8, 8, 2, 8, 4 and 4 ways; 32-, 16-
    and 64-row blocks; three end in a partial strip): its counters are reset
    by the kernel, so a captured call replays with every replay equal to the
    eager call, eager work between."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=13 + M)
    ext = ng.extension()
    assert ext.gemm_workspace_bytes(M, K_, N, g, 6, None)[1] > 0  # this plan splits K
    eager = ng.gemm(Xd, qw)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ng.gemm(Xd, qw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ng.gemm(Xd, qw)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ng.gemm(Xd, qw)
        torch.cuda.synchronize()
    assert rms_err(host(eager), oracle_y(X, packed, scales, K_, g)) <= RMS_TOL


@pytest.mark.parametrize("M", [128, 512, 2048])
@pytest.mark.parametrize("K_,N", [(4096, 14336), (14336, 4096)])
def test_prefill_configs_sampled_rows(M, K_, N):
    """The prefill config (M = 128, 512, 2048 at 4096 x 14336 and 14336 x 4096)
    at full size; the oracle checks 12 sampled rows (first, last, both sides
    of every 128-row tile edge it hits, random)."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=300 + M + N)
    y = host(ng.gemm(Xd, qw))
    rng = np.random.default_rng(M)
    rows = sorted(set([0, 1, 127, M - 1] + [int(r) for r in rng.integers(0, M, size=8)]))
    rows = [r for r in rows if r < M]
    ref = oracle_y_rows(X, rows, packed, scales, K_, 128)
    assert rms_err(y[rows], ref) <= RMS_TOL
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("M", [128, 512, 2048])
@pytest.mark.parametrize("K_,N", [(4096, 14336), (14336, 4096)])
def test_prefill_configs_whole_output(M, K_, N):
    """Every output of the prefill configs, both versions, against an fp32
    product on the GPU of the dequant kernel's weights (bit-exact with the
    oracle's dequantize, tests/test_dequant.py): a wrong tile, split or row
    block anywhere fails."""
    _, _, _, Xd, qw = synthetic(M, K_, N, 128, seed=300 + M + N)
    ref = Xd.float() @ ng.dequant(qw).float()
    rms = ref.pow(2).mean().sqrt()
    for version in (6, 7):
        y = ng.gemm(Xd, qw, version=version).float()
        assert torch.isfinite(y).all()
        assert float((y - ref).abs().max() / rms) <= RMS_TOL, version


@pytest.mark.parametrize("K_,N", [(4096, 14336), (14336, 4096)])
def test_prefill_m2048_whole_output_against_the_oracle(K_, N):
    """The bench's prefill points (M = 2048 at both config-4 shapes), every
    output of both versions against the CPU oracle's reference path
    (dequantize, fp32 matmul, fp16; ~3-5 s a shape on the host's cores)."""
    X, packed, scales, Xd, qw = synthetic(2048, K_, N, 128, seed=2048 + K_)
    ref = oracle_y(X, packed, scales, K_, 128)
    for version in (6, 7):
        y = host(ng.gemm(Xd, qw, version=version))
        assert np.all(np.isfinite(y)), version
        assert rms_err(y, ref) <= RMS_TOL, version


def test_gemm_is_deterministic():
    _, _, _, Xd, qw = synthetic(257, 2048, 1024, 128, seed=5)
    a = ng.gemm(Xd, qw)
    b = ng.gemm(Xd, qw)
    assert torch.equal(a, b)


def test_golden_vectors():
    z = np.load(GOLDEN)
    for name in sorted({k.split("/")[0] for k in z.files if not k.startswith("sweep")}):
        M, K_, N, g, _ = z[f"{name}/meta"].tolist()
        qw = to_dev_qw(z[f"{name}/qweight"], z[f"{name}/scales"], K_, N, g)
        X = torch.from_numpy(z[f"{name}/X"].view(np.float16).copy()).cuda()
        ref = z[f"{name}/Y"].view(np.float16).astype(np.float32)
        for version in (6, 7):
            assert rms_err(host(ng.gemm(X, qw, version=version)), ref) <= RMS_TOL, (name, version)


def test_empty_batch():
    _, _, _, Xd, qw = quantized(4, 256, 128, 128, seed=8)
    assert ng.gemm(Xd[:0], qw).shape == (0, 128)


def test_gemm_rejects_bad_version():
    _, _, _, Xd, qw = quantized(16, 256, 128, 128, seed=9)
    with pytest.raises(RuntimeError):
        ng.gemm(Xd, qw, version=5)


@pytest.mark.parametrize("M", [9, 16, 24, 32, 33, 64, 100, 128, 129])
@pytest.mark.parametrize("K_,N,g", [(4096, 1024, 128), (14336, 512, 128), (1024, 260, 64)])
def test_small_batch_handover(M, K_, N, g):
    """M <= 128 runs the weight-streaming kernel (32-row blocks, split over K
    when K is long), M = 129 the tile kernel; both against the oracle."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M * 3 + N)
    ref = oracle_y(X, packed, scales, K_, g)
    for version in (6, 7):
        y = host(ng.gemm(Xd, qw, version=version))
        assert rms_err(y, ref) <= RMS_TOL, version
        assert rel_err(y, ref) < REL_TOL, version


@pytest.mark.parametrize("M,K_,N", [(M, K_, N) for M in (100, 128)
                                    for K_, N in ((4096, 14336), (14336, 4096), (8192, 8192))]
                         + [(100, 14336, 4100), (47, 8192, 8200), (65, 4096, 14340),
                            (40, 4096, 28672), (64, 8192, 14336)])
def test_small_batch_tiles(M, K_, N):
    """Batches of 33..128 rows over large weights (32-row weight passes of
    48 MiB or more, where one 64-row block would not make one round of the
    CUs) take 64-row producer/consumer tiles split over K instead of
    streaming: every output, both versions (the same plan, so the same
    bits), repeated calls bit-identical, against an fp32 product of the
    dequant kernel's weights on the GPU.  Three shapes end in partial row
    and column tiles."""
    ext = ng.extension()
    assert not ext.gemm_streams(M, K_, N, 128)
    _, _, _, Xd, qw = synthetic(M, K_, N, 128, seed=400 + M + N)
    ref = Xd.float() @ ng.dequant(qw).float()
    rms = ref.pow(2).mean().sqrt()
    y6 = ng.gemm(Xd, qw, version=6)
    assert torch.equal(ng.gemm(Xd, qw, version=7), y6)
    assert torch.equal(ng.gemm(Xd, qw, version=6), y6)
    assert torch.equal(ng.matmul(Xd, qw), y6)
    y = y6.float()
    assert torch.isfinite(y).all()
    assert float((y - ref).abs().max() / rms) <= RMS_TOL


@pytest.mark.parametrize("M,K_,N", [(129, 4096, 4096), (192, 4096, 4096), (256, 4096, 4096),
                                    (160, 4096, 6144), (200, 6144, 4096), (256, 4096, 6144)])
def test_mid_k_split(M, K_, N):
    """4096 <= K < 8192 with at most 160 64-row tiles splits K 4 ways (all
    but 256 x 4096 x 6144, whose 192 tiles run unsplit; 200 x 6144 x 4096
    has a row tail and 24 k steps per split): every output against an fp32
    product of the dequant kernel's weights, repeated calls bit-identical."""
    _, _, _, Xd, qw = synthetic(M, K_, N, 128, seed=500 + M + N)
    ref = Xd.float() @ ng.dequant(qw).float()
    rms = ref.pow(2).mean().sqrt()
    y = ng.gemm(Xd, qw)
    assert torch.equal(ng.gemm(Xd, qw), y)
    assert torch.isfinite(y.float()).all()
    assert float((y.float() - ref).abs().max() / rms) <= RMS_TOL


@pytest.mark.parametrize("M,K_,N", [(64, 14336, 4096), (129, 4096, 4096), (160, 14336, 512),
                                    (24, 14336, 1024)])
def test_split_plans_repeat_their_bits(M, K_, N):
    """Every split plan's last-arriver sum, called 300 times back to back
    (64-row tiles split 8 ways, 4096 <= K < 8192 split 4 ways, 128-row tiles
    split 4 ways, the streaming kernel's split K): identical bits each time,
    so no call reads a partial before it is complete."""
    _, _, _, Xd, qw = synthetic(M, K_, N, 128, seed=900 + M)
    ext = ng.extension()
    assert ext.gemm_workspace_bytes(M, K_, N, 128, 6, None)[1] > 0  # a split plan
    first = ng.gemm(Xd, qw)
    outs = [ng.gemm(Xd, qw) for _ in range(300)]
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(y, first)


def test_small_batch_split_k_is_deterministic():
    _, _, _, Xd, qw = synthetic(24, 14336, 1024, 128, seed=77)
    ys = [ng.gemm(Xd, qw) for _ in range(4)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@pytest.mark.parametrize("M,K_,N", [(140, 8192, 640), (200, 14336, 256), (300, 8192, 1024),
                                    (133, 8192, 130)])
def test_tile_kernel_split_k(M, K_, N):
    """Few output tiles over a long K split the reduction across workgroups
    (deterministic last-arriver sum); both versions against the oracle."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=M + K_ + N)
    ref = oracle_y(X, packed, scales, K_, 128)
    for version in (6, 7):
        ys = [ng.gemm(Xd, qw, version=version) for _ in range(3)]
        for y in ys[1:]:
            assert torch.equal(y, ys[0]), version
        assert rms_err(host(ys[0]), ref) <= RMS_TOL, version


@pytest.mark.parametrize("M", [9, 12, 16])
@pytest.mark.parametrize("K_,N,g", [(4096, 14336, 128), (2048, 12292, 64)])
def test_sixteen_row_strip_blocks(M, K_, N, g):
    """9 <= M <= 16 over a short K and a wide N runs the decode GEMV's strip
    kernel with 16-row blocks and the activations staged in LDS (128 KiB at
    K = 4096), also with a 4-column strip tail (N = 12292); both versions
    against the oracle, and repeatable."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M + K_ + N)
    ref = oracle_y(X, packed, scales, K_, g)
    for version in (6, 7):
        y = ng.gemm(Xd, qw, version=version)
        assert torch.equal(y, ng.gemm(Xd, qw, version=version))
        assert rms_err(host(y), ref) <= RMS_TOL, version
        assert rel_err(host(y), ref) < REL_TOL, version


@pytest.mark.parametrize("M,K_,N,g", [(129, 320, 132, 64), (257, 576, 260, 64), (1000, 128, 4100, 128),
                                      (300, 8256, 516, 64), (192, 4096, 640, 128)])
def test_producer_consumer_kernel_edges(M, K_, N, g):
    """Shapes for the 64-k producer/consumer kernel: row and column tails of
    its 64/128-row, 128-column tiles, odd numbers of 64-k steps, group 64 and
    a K split (K >= 8192)."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M + K_ + N)
    ref = oracle_y(X, packed, scales, K_, g)
    for version in (6, 7):
        ys = [ng.gemm(Xd, qw, version=version) for _ in range(2)]
        assert torch.equal(ys[0], ys[1]), version
        assert rms_err(host(ys[0]), ref) <= RMS_TOL, version
        assert rel_err(host(ys[0]), ref) < REL_TOL, version


@pytest.mark.parametrize("M,K_,N,g", [(1024, 256, 14336, 128), (4096, 512, 4096, 64),
                                      (1100, 384, 12000, 128), (2048, 256, 14336, 128),
                                      (1024, 320, 14336, 64), (4000, 256, 4000, 64)])
def test_large_tile_kernel(M, K_, N, g):
    """Version 6 runs 256 x 256 tiles from M = 1024 when the grid is one round
    over the CUs, at least 7/8 full: 224 tiles at 1024 x 14336, 256 at
    4096 x 4096, and with row and column tails 235 at 1100 x 12000 and 256
    at 4000 x 4000; 2048 x 14336 (448 tiles) runs the twelve-wave 256 x 128
    kernel instead.  Every kernel sums each output over k in the same order,
    so version 6 and version 7 (128 x 128) agree to the bit."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M + K_ + N)
    y6 = ng.gemm(Xd, qw, version=6)
    y7 = ng.gemm(Xd, qw, version=7)
    assert torch.equal(y6, y7)
    assert torch.equal(ng.gemm(Xd, qw, version=6), y6)
    ref = oracle_y(X, packed, scales, K_, g)
    assert rms_err(host(y6), ref) <= RMS_TOL
    assert rel_err(host(y6), ref) < REL_TOL


@pytest.mark.parametrize("M,K_,N,g", [(2100, 256, 3500, 128), (2048, 320, 4096, 64),
                                      (2049, 448, 3584, 64)])
def test_twelve_wave_kernel(M, K_, N, g):
    """Version 6 runs 256 x 128 tiles with eight consumer waves from M = 2048
    when that grid makes whole rounds of the CUs (the last at least 7/8 full)
    and the 256 x 256 kernel does not: with row and column tails (252 tiles
    at 2100 x 3500), an odd number of 64-k steps with group 64 (256 tiles),
    and a single-row tail (252 tiles at 2049 x 3584).  Its k order is the
    128 x 128 kernel's, so version 6 and version 7 agree to the bit."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, g, seed=M + K_ + N)
    y6 = ng.gemm(Xd, qw, version=6)
    y7 = ng.gemm(Xd, qw, version=7)
    assert torch.equal(y6, y7)
    assert torch.equal(ng.gemm(Xd, qw, version=6), y6)
    ref = oracle_y(X, packed, scales, K_, g)
    assert rms_err(host(y6), ref) <= RMS_TOL
    assert rel_err(host(y6), ref) < REL_TOL


def _offset_copy(t: torch.Tensor, elems: int) -> torch.Tensor:
    """A contiguous copy of ``t`` starting ``elems`` elements into a larger buffer."""
    buf = torch.empty(t.numel() + elems, dtype=t.dtype, device=t.device)
    out = buf[elems:].view(t.shape)
    out.copy_(t)
    return out


@pytest.mark.parametrize("M,K_,N", [(300, 512, 260), (600, 1024, 512)])
def test_gemm_under_aligned_weights(M, K_, N):
    """Weights only 8-byte (packed) / 4-byte (scales) aligned cannot take the
    producer/consumer kernel's 16-byte loads and run the tile kernel; both
    sum every output over k in the same order, so without a K split the bits
    agree."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=M + N)
    qw_off = ng.QuantizedWeight(_offset_copy(qw.qweight, 2), _offset_copy(qw.scales, 2),
                                qw.group_size, qw.K, qw.N)
    assert qw_off.qweight.data_ptr() % 16 == 8
    y = ng.gemm(Xd, qw)
    y_off = ng.gemm(Xd, qw_off)
    assert torch.equal(y, y_off)
    assert rms_err(host(y_off), oracle_y(X, packed, scales, K_, 128)) <= RMS_TOL


@pytest.mark.parametrize("M,K_,N", [(160, 14336, 512), (64, 14336, 4096), (129, 4096, 4096)])
def test_split_k_gemm_replays_in_a_graph(M, K_, N):
    """The producer/consumer kernel's K split (counters reset by the kernel
    itself, no memset) is graph-capturable; every replay matches eager, with
    eager work between replays.  Shapes: 128-row tiles split 4 ways over a
    long K; a small batch on 64-row tiles split 8 ways; 4096 <= K < 8192 with
    few tiles, split 4 ways."""
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=11)
    ext = ng.extension()
    assert ext.gemm_workspace_bytes(M, K_, N, 128, 6, None)[1] > 0  # this plan splits K
    eager = ng.gemm(Xd, qw)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ng.gemm(Xd, qw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ng.gemm(Xd, qw)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ng.gemm(Xd, qw)
        torch.cuda.synchronize()
    assert rms_err(host(eager), oracle_y(X, packed, scales, K_, 128)) <= RMS_TOL


def test_split_k_sum_into_under_aligned_output():
    """The C ABI asks only 2-byte alignment of Y.  The split-K tile sum stores
    4 columns at once when Y allows it and element by element otherwise; both
    give the bits of the call into a freshly allocated Y."""
    M, K_, N = 160, 14336, 512
    X, packed, scales, Xd, qw = synthetic(M, K_, N, 128, seed=11)
    ext = ng.extension()
    ws_bytes, counter_bytes = ext.gemm_workspace_bytes(M, K_, N, 128, 6, None)
    assert counter_bytes > 0  # this plan splits K
    want = ng.gemm(Xd, qw)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=Xd.device)
    buf = torch.zeros(M * N + 8, dtype=torch.float16, device=Xd.device)
    for start in (1, 2, 4):  # Y 2-, 4- and 8-byte aligned
        y = buf[start:start + M * N].view(M, N)
        assert y.data_ptr() % 8 == 2 * start % 8
        rc = ext.gemm(Xd.data_ptr(), M, K_, qw.qweight.data_ptr(), qw.qweight.shape[0], N,
                      qw.scales.data_ptr(), qw.scales.shape[0], qw.scales.shape[1], 128, 6,
                      y.data_ptr(), ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, ext.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y, want), start
        assert buf[:start].eq(0).all() and buf[start + M * N:].eq(0).all(), start
        buf.zero_()
