"""Parity of the decode GEMV (versions 0-4) with the reference path.

The checker is the CPU oracle's dequantize-then-fp32-matmul (the reference's
reference_matmul, python/nibblegemm/quant.py:207-215).  Two bounds are
asserted on every comparison:

* ``max|y - ref| <= 1e-2 * rms(ref)`` (RMS_TOL);
* the reference suite's ``max|y - ref| / mean|ref| < 5e-2`` (REL_TOL,
  tests/test_gemv.py:29 there).

The streaming kernels (the strip kernel for the default plan up to K = 8192,
the split kernel beyond it and for explicit overrides) accumulate exact fp16 x
fp16 products in fp32 on the matrix cores (v_mfma_f32_16x16x32_f16) and scale
fp32 group sums, so their error against the oracle is fp32 summation order plus
the final fp16 rounding: ~1e-3 of RMS at most.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from cases import DECODE_SHAPES, host, oracle_y, quantized, rel_err, rms_err, synthetic, to_dev_qw

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-2
REL_TOL = 5e-2
VERSIONS = [0, 1, 2, 3, 4]
SHAPES = [(512, 256), (256, 132)]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w4a16_golden.npz")


@pytest.mark.parametrize("version", VERSIONS)
@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("K,N", SHAPES)
def test_gemv_matches_reference(version, M, group_size, K, N):
    X, packed, scales, Xd, qw = quantized(M, K, N, group_size)
    y = ng.gemv(Xd, qw, version=version)
    assert y.shape == (M, N) and y.dtype == torch.float16
    ref = oracle_y(X, packed, scales, K, group_size)
    assert rms_err(host(y), ref) <= RMS_TOL
    assert rel_err(host(y), ref) < REL_TOL


@pytest.mark.parametrize("M", [1, 3, 5, 8])
@pytest.mark.parametrize("K,N", [(4096, 4096), (1024, 4100), (2048, 260), (128, 4)])
def test_gemv_synthetic_distributions(M, K, N):
    X, packed, scales, Xd, qw = synthetic(M, K, N, 128, seed=M * 7 + N)
    y = host(ng.gemv(Xd, qw))
    ref = oracle_y(X, packed, scales, K, 128)
    assert rms_err(y, ref) <= RMS_TOL


@pytest.mark.parametrize("K,N", DECODE_SHAPES)
def test_decode_configs_full_size(K, N):
    """The decode configs (M = 1, g = 128) at their real shapes."""
    X, packed, scales, Xd, qw = synthetic(1, K, N, 128, seed=K + N)
    y = host(ng.gemv(Xd, qw))
    ref = oracle_y(X, packed, scales, K, 128)
    assert rms_err(y, ref) <= RMS_TOL
    assert rel_err(y, ref) < REL_TOL


@pytest.mark.parametrize("M", [2, 4, 8])
def test_small_batch_config_gemv_leg(M):
    """The small-batch config at M <= 8 (the GEMV side of the handover)."""
    X, packed, scales, Xd, qw = synthetic(M, 4096, 14336, 128, seed=100 + M)
    y = host(ng.matmul(Xd, qw))
    assert rms_err(y, oracle_y(X, packed, scales, 4096, 128)) <= RMS_TOL


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("K,N", SHAPES)
def test_gemv_versions_agree(M, group_size, K, N):
    _, _, _, Xd, qw = quantized(M, K, N, group_size, seed=1)
    base = host(ng.gemv(Xd, qw, version=0))
    for version in VERSIONS[1:]:
        assert rel_err(host(ng.gemv(Xd, qw, version=version)), base) < REL_TOL, f"v{version}"


SPLIT_K, SPLIT_N, SPLIT_G = 1024, 256, 64
SPLIT_TOL = 2e-2


@pytest.mark.parametrize("M", [1, 4, 8])
@pytest.mark.parametrize("splits", [1, 4, 16])
def test_gemv_splitk_is_invariant(M, splits):
    X, packed, scales, Xd, qw = quantized(M, SPLIT_K, SPLIT_N, SPLIT_G, seed=2)
    y = host(ng.gemv(Xd, qw, version=4, splits=splits))
    single = host(ng.gemv(Xd, qw, version=3))
    assert rel_err(y, single) < SPLIT_TOL
    assert rms_err(y, oracle_y(X, packed, scales, SPLIT_K, SPLIT_G)) <= RMS_TOL


def test_v3_is_v4_with_one_split():
    _, _, _, Xd, qw = quantized(4, SPLIT_K, SPLIT_N, SPLIT_G, seed=3)
    assert torch.equal(ng.gemv(Xd, qw, version=4, splits=1), ng.gemv(Xd, qw, version=3))


@pytest.mark.parametrize("threads", [32, 64, 128, 256, 512, 1024])
def test_block_threads_override(threads):
    M = 1 if threads == 1024 else 2
    X, packed, scales, Xd, qw = synthetic(M, 2048, 1280, 128, seed=threads)
    y = host(ng.gemv(Xd, qw, block_threads=threads))
    assert rms_err(y, oracle_y(X, packed, scales, 2048, 128)) <= RMS_TOL


def test_split_k_is_deterministic_and_counters_return_to_zero():
    # 14336 x 4096 is split over workgroups by the default plan (112 groups);
    # 300 back-to-back calls: no call's last arriver reads an incomplete partial
    _, _, _, Xd, qw = synthetic(2, 14336, 4096, 128, seed=4)
    ys = [ng.gemv(Xd, qw) for _ in range(300)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    from nibblegemm_amd import ops

    stream = torch.cuda.current_stream().cuda_stream
    counter_bytes = ng.extension().gemv_workspace_bytes(2, 14336, 4096, 128, 4, 0, 0, stream)[1]
    assert counter_bytes > 0
    buf = ops._workspaces[(Xd.device.index, stream, 0, counter_bytes)]
    assert int(buf[:counter_bytes].count_nonzero()) == 0


@pytest.mark.parametrize("version", [3, 4])
def test_gemv_rejects_m_above_8(version):
    _, _, _, Xd, qw = quantized(9, 256, 132, 128, seed=4)
    with pytest.raises(RuntimeError):
        ng.gemv(Xd, qw, version=version)


@pytest.mark.parametrize("version", [0, 1, 2])
def test_low_versions_accept_m_above_8(version):
    X, packed, scales, Xd, qw = quantized(19, 256, 132, 128, seed=5)
    y = host(ng.gemv(Xd, qw, version=version))
    assert rms_err(y, oracle_y(X, packed, scales, 256, 128)) <= RMS_TOL


def test_matmul_dispatches_to_gemv_below_the_crossover():
    _, _, _, Xd, qw = quantized(ng.DECODE_MAX_M, 512, 256, 128, seed=5)
    assert torch.equal(ng.matmul(Xd, qw), ng.gemv(Xd, qw, version=4))


def test_matmul_rejects_k_mismatch():
    _, _, _, _, qw = quantized(1, 512, 256, 128, seed=6)
    X = torch.randn(1, 256, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):
        ng.matmul(X, qw)


def test_gemv_input_errors_raise_runtime_error():
    _, _, _, Xd, qw = quantized(1, 256, 128, 128, seed=7)
    with pytest.raises(RuntimeError):
        ng.gemv(Xd.float(), qw)
    strided = torch.randn(256, 2, device="cuda", dtype=torch.float16).t()  # [2, 256], not contiguous
    with pytest.raises(RuntimeError):
        ng.gemv(strided, qw)


def test_empty_batch_and_empty_reduction():
    _, _, _, Xd, qw = quantized(1, 256, 128, 128, seed=8)
    assert ng.gemv(Xd[:0], qw).shape == (0, 128)
    qw0 = ng.QuantizedWeight(torch.zeros((0, 128), dtype=torch.int32, device="cuda"),
                             torch.zeros((0, 128), dtype=torch.float16, device="cuda"), 128, 0, 128)
    y = ng.gemv(torch.zeros((2, 0), dtype=torch.float16, device="cuda"), qw0)
    assert y.shape == (2, 128) and int(y.count_nonzero()) == 0


def test_golden_vectors():
    z = np.load(GOLDEN)
    for name in sorted({k.split("/")[0] for k in z.files if not k.startswith("sweep")}):
        M, K, N, g, _ = z[f"{name}/meta"].tolist()
        if M > ng.DECODE_MAX_M:
            continue
        qw = to_dev_qw(z[f"{name}/qweight"], z[f"{name}/scales"], K, N, g)
        X = torch.from_numpy(z[f"{name}/X"].view(np.float16).copy()).cuda()
        ref = z[f"{name}/Y"].view(np.float16).astype(np.float32)
        for version in VERSIONS:
            assert rms_err(host(ng.gemv(X, qw, version=version)), ref) <= RMS_TOL, (name, version)


def test_graph_capture_replays_match_eager():
    """The single-launch split-K kernel is graph-capturable; every replay
    matches eager (replays interleaved with eager work)."""
    X, packed, scales, Xd, qw = synthetic(1, 4096, 14336, 128, seed=9)
    eager = ng.gemv(Xd, qw)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ng.gemv(Xd, qw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ng.gemv(Xd, qw)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ng.gemv(Xd, qw)  # eager work between replays
        torch.cuda.synchronize()


def test_gemv_timeline():
    """The decode GEMV's in-kernel timeline (nibble_gemv_timeline): every
    wave of every workgroup with a strip records its 7 points in order and
    its placement; the outputs keep their bits (packed and strip-major); a
    buffer too small for the launch is refused before anything runs; M > 1
    launches leave the buffer alone."""
    ext = ng.extension()
    _, _, _, Xd, qw = synthetic(1, 4096, 14336, 128, seed=12)
    sm = ng.to_strip_major(qw, 64)
    want, want_sm = ng.gemv(Xd, qw), ng.matmul(Xd, sm)
    strips, waves = 224, 4  # 64-column strips, 4 waves (the decode plan at this shape)
    stamps = torch.zeros(strips * waves * 8, dtype=torch.int64, device="cuda")
    try:
        assert ext.gemv_timeline(stamps.data_ptr(), stamps.numel() * 8) == 0
        for fn, ref in ((lambda: ng.gemv(Xd, qw), want), (lambda: ng.matmul(Xd, sm), want_sm)):
            stamps.zero_()
            assert torch.equal(fn(), ref)
            torch.cuda.synchronize()
            t = stamps.view(strips, waves, 8).cpu().numpy()
            times = t[:, :, :7]
            assert (times > 0).all()
            assert (np.diff(times, axis=2) >= 0).all()
            assert (times[:, :, 6] - times[:, :, 0]).max() < 100_000  # < 1 ms at 100 MHz
            xcc = (t[:, :, 7] >> 32) & 0xF
            assert set(np.unique(xcc).tolist()) <= set(range(8))
            assert ((t[:, :, 7] >> 40) == np.arange(strips)[:, None]).all()
            assert (((t[:, :, 7] >> 36) & 0xF) == np.arange(waves)[None, :]).all()
        stamps.zero_()
        _, _, _, X2, _ = synthetic(2, 4096, 14336, 128, seed=13)
        ng.gemv(X2, qw)
        torch.cuda.synchronize()
        assert int(stamps.abs().sum()) == 0
        assert ext.gemv_timeline(stamps.data_ptr(), 1024) == 0
        with pytest.raises(RuntimeError, match="timeline"):
            ng.gemv(Xd, qw)
    finally:
        assert ext.gemv_timeline(None, 0) == 0
    assert torch.equal(ng.gemv(Xd, qw), want)
