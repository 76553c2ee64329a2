"""Strip-major weights for the decode GEMV (``nibble_pack_strip_major``,
``nibble_gemv_w4a16_strip_major``, ``ops.to_strip_major``).

* The layout: ``Wt[s][r][j] == Wq[r][s * SW + j]`` and ``St[s][g][j] ==
  S[g][s * SW + j]``, checked element by element against the packed arrays
  (CPU), and the device pack kernel bit for bit against that definition.
* The GEMV on strip-major weights against the C oracle at every decode shape
  and M = 1..8 (north-star bound ``max|y - ref| <= 1e-2 rms(ref)``), and
  against the packed-layout GEMV of the same weight.
* Its epilogues and RMSNorm prologue have the bits of the separate fp16 ops
  run after the plain strip-major product; graph replays repeat eager bits.
* Host-side rejections happen before any HIP call (CPU).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import ops, quant
import oracle as O
from cases import DECODE_SHAPES, host, oracle_y, rms_err, synthetic

OK, INVALID, UNSUPPORTED = 0, 1, 2
P = 1 << 20  # aligned, never dereferenced
RMS_TOL = 1e-2


# ---------------------------------------------------------------- CPU tier

@pytest.mark.parametrize("sw", [16, 32, 64])
def test_layout_definition_element_by_element(sw):
    K, N, g = 256, 192, 64
    rng = np.random.default_rng(sw)
    packed = rng.integers(-2**31, 2**31, size=(K // 8, N), dtype=np.int64).astype(np.int32)
    scales = rng.standard_normal((K // g, N)).astype(np.float16)
    qw = ng.QuantizedWeight(torch.from_numpy(packed), torch.from_numpy(scales), g, K, N)
    sm = quant.strip_major(qw, sw)
    assert tuple(sm.qweight.shape) == (N // sw, K // 8, sw)
    assert tuple(sm.scales.shape) == (N // sw, K // g, sw)
    wt, st = sm.qweight.numpy(), sm.scales.numpy()
    for s in range(N // sw):
        for j in range(sw):
            n = s * sw + j
            assert np.array_equal(wt[s, :, j], packed[:, n])
            assert np.array_equal(st[s, :, j].view(np.uint16), scales[:, n].view(np.uint16))
    assert sm.weight_bytes == qw.weight_bytes


def test_layout_definition_rejects_bad_widths():
    qw = ng.QuantizedWeight(torch.zeros(4, 48, dtype=torch.int32),
                            torch.zeros(1, 48, dtype=torch.float16), 32, 32, 48)
    with pytest.raises(ValueError, match="strip_cols must be one of"):
        quant.strip_major(qw, 24)
    with pytest.raises(ValueError, match="not a multiple"):
        quant.strip_major(qw, 32)


@pytest.mark.parametrize("K,N,g,want", [
    (14336, 4096, 128, 16),   # down projection: few 32-column strips, long K
    (4096, 1024, 128, 16),    # k / v
    (4096, 4096, 128, 16),   # short K, few columns: 16-column strips measured faster
    (4096, 6144, 128, 32),
    (4096, 14336, 128, 64),
    (4096, 28672, 128, 64),
    (8192, 8192, 128, 32),
    (4096, 1024, 64, 32),     # 16-column strips need g = 128
    (4096, 80, 128, 16),
    (4096, 40, 128, 0),
    (4096, 48, 64, 0),
    (100, 128, 128, 0),       # K not a multiple of g
])
def test_recommended_strip_width(K, N, g, want):
    assert ng.strip_major_cols(K, N, g) == want


def pack(ext, K=256, N=128, g=128, sw=32, wq_rows=None, s_rows=None, s_cols=None, ptr=P, out=None):
    wq_rows = K // 8 if wq_rows is None else wq_rows
    s_rows = K // g if s_rows is None else s_rows
    s_cols = N if s_cols is None else s_cols
    out = (8 * P, 16 * P) if out is None else out
    return ext.pack_strip_major(ptr, wq_rows, N, ptr + P, s_rows, s_cols, g, sw, out[0], out[1],
                                None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(sw=24), "strip_cols must be 16, 32 or 64"),
    (dict(N=96, sw=64), "not a multiple of strip_cols"),
    (dict(g=64, sw=16), "16-column strips need group_size 128"),
    (dict(s_rows=3), "scale rows"),
    (dict(s_cols=132), "scale columns"),
    (dict(g=32), "group_size"),
    (dict(ptr=P + 8), "16-byte aligned"),
    (dict(out=(P, 16 * P)), "must not overlap"),
    (dict(ptr=0), "null"),
])
def test_pack_rejections(kwargs, needle):
    ext = ng.extension()
    assert pack(ext, **kwargs) == INVALID
    assert needle in ext.last_error()


def sm_gemv(ext, M=1, K=256, N=128, g=128, sw=32, epilogue=0, bias=P, norm=None, eps=1e-5,
            x_cols=None, ptr=P):
    x_cols = K if x_cols is None else x_cols
    return ext.gemv_strip_major(ptr, M, x_cols, ptr, ptr, K, N, g, sw, epilogue, bias, norm, eps,
                                ptr, None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(M=9), "M <= 8"),
    (dict(x_cols=512), "disagree with K"),
    (dict(K=200), "multiple of group_size"),
    (dict(sw=48), "strip_cols must be 16, 32 or 64"),
    (dict(N=96, sw=64), "not a multiple of strip_cols"),
    (dict(g=64, sw=16), "16-column strips need group_size 128"),
    (dict(epilogue=3), "epilogue"),
    (dict(epilogue=2, sw=16), "at least 32 columns"),
    (dict(epilogue=1, bias=None), "null bias"),
    (dict(norm=P, K=16384 + 128), "K <= 16384"),
    (dict(norm=P, M=8, K=8192), "above 64 KiB"),
    (dict(norm=P + 8), "norm weight must be 16-byte aligned"),
    (dict(norm=P, eps=float("nan")), "norm eps"),
    (dict(ptr=P + 8), "aligned"),
    (dict(ptr=0), "null"),
])
def test_strip_major_gemv_rejections(kwargs, needle):
    ext = ng.extension()
    assert sm_gemv(ext, **kwargs) == INVALID
    assert needle in ext.last_error()


def test_strip_major_gemv_empty_batch_is_a_no_op():
    ext = ng.extension()
    assert sm_gemv(ext, M=0, ptr=0) == OK


def test_host_strip_major_weights_are_refused():
    sm = quant.strip_major(ng.QuantizedWeight(torch.zeros(32, 64, dtype=torch.int32),
                                              torch.zeros(2, 64, dtype=torch.float16), 128, 256,
                                              64), 32)
    with pytest.raises(RuntimeError, match="GPU"):
        ng.matmul(torch.zeros(1, 256, dtype=torch.float16), sm)


# ---------------------------------------------------------------- GPU tier

def strip_case(M, K, N, g, sw=0, seed=0):
    X, packed, scales, Xd, qw = synthetic(M, K, N, g, seed=seed)
    return X, packed, scales, Xd, qw, ng.to_strip_major(qw, sw)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,g,sw", [(256, 128, 128, 16), (256, 128, 64, 32), (1024, 448, 128, 64),
                                      (14336, 4096, 128, 16), (4096, 14336, 128, 64)])
def test_pack_kernel_is_the_layout_definition(K, N, g, sw):
    _, _, _, _, qw = synthetic(1, K, N, g, seed=K + sw)
    dev = ng.to_strip_major(qw, sw)
    ref = quant.strip_major(qw.to("cpu"), sw)
    assert dev.strip_cols == sw and (dev.K, dev.N, dev.group_size) == (K, N, g)
    assert torch.equal(dev.qweight.cpu(), ref.qweight)
    assert torch.equal(dev.scales.cpu().view(torch.int16), ref.scales.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", DECODE_SHAPES + [(4096, 6144), (4096, 28672)])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_decode_shapes_match_the_oracle(K, N, M):
    X, packed, scales, Xd, qw, sm = strip_case(M, K, N, 128, seed=M + K)
    assert sm.strip_cols == ng.strip_major_cols(K, N, 128)
    y = ng.matmul(Xd, sm)
    assert y.shape == (M, N) and y.dtype == torch.float16
    assert rms_err(host(y), oracle_y(X, packed, scales, K, 128)) <= RMS_TOL
    # the packed-layout GEMV of the same weight: equal up to summation order
    # (a one-ulp fp16 difference at the largest outputs is ~2e-3 of rms)
    assert rms_err(host(y), host(ng.matmul(Xd, qw))) <= 5e-3


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,g,sw", [(1, 256, 64, 128, 16), (4, 512, 96, 64, 32),
                                        (7, 1024, 192, 128, 64), (8, 14336, 512, 128, 16),
                                        (3, 2048, 1024, 64, 64), (2, 12288, 256, 128, 32)])
def test_every_width_matches_the_oracle(M, K, N, g, sw):
    X, packed, scales, Xd, _, sm = strip_case(M, K, N, g, sw, seed=sw + M)
    assert rms_err(host(ng.matmul(Xd, sm)), oracle_y(X, packed, scales, K, g)) <= RMS_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,sw", [(1, 4096, 1024, 16), (8, 4096, 4096, 32), (3, 4096, 14336, 64)])
def test_bias_epilogue_is_the_separate_add(M, K, N, sw):
    _, _, _, Xd, _, sm = strip_case(M, K, N, 128, sw, seed=11)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(N)) * 0.5).half().cuda()
    assert torch.equal(ng.matmul_bias(Xd, sm, bias), ng.matmul(Xd, sm) + bias)
    # an fp32 bias promotes, as for the packed weight
    b32 = bias.float()
    assert torch.equal(ng.matmul_bias(Xd, sm, b32), ng.matmul(Xd, sm) + b32)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,Nh,sw", [(1, 4096, 14336, 64), (5, 1024, 512, 32)])
def test_swiglu_epilogue_is_the_fp16_composition(M, K, Nh, sw):
    _, _, _, Xd, gate = synthetic(M, K, Nh, 128, seed=1)
    _, _, _, _, up = synthetic(M, K, Nh, 128, seed=2)
    sm = ng.to_strip_major(ng.interleave_swiglu(gate, up), sw)
    fused = ng.matmul_swiglu(Xd, sm)
    gate_y, up_y = quant.split_swiglu(ng.matmul(Xd, sm))
    assert fused.shape == (M, Nh)
    assert torch.equal(fused, torch.nn.functional.silu(gate_y) * up_y)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,Nh", [(1, 4096, 1024), (3, 4096, 512)])
def test_swiglu_on_default_16_column_strips_composes(M, K, Nh):
    """A gate|up weight whose recommended strip width is 16 columns (N <= 2048)
    cannot take the SwiGLU epilogue (a strip holds half a gate|up block pair);
    matmul_swiglu and rmsnorm_matmul(swiglu=True) compose the same fp16
    arithmetic from the plain strip-major product instead of refusing."""
    _, _, _, Xd, gate = synthetic(M, K, Nh, 128, seed=3)
    _, _, _, _, up = synthetic(M, K, Nh, 128, seed=4)
    sm = ng.to_strip_major(ng.interleave_swiglu(gate, up))
    assert sm.strip_cols == 16
    gate_y, up_y = quant.split_swiglu(ng.matmul(Xd, sm))
    want = torch.nn.functional.silu(gate_y) * up_y
    assert torch.equal(ng.matmul_swiglu(Xd, sm), want)
    w = (torch.rand(K, generator=torch.Generator().manual_seed(9)) + 0.5).half().cuda()
    from nibblegemm_amd.glue import rmsnorm  # noqa: PLC0415

    g2, u2 = quant.split_swiglu(ng.matmul(rmsnorm(Xd, w, 1e-5), sm))
    assert torch.equal(ng.rmsnorm_matmul(Xd, w, sm, 1e-5, swiglu=True),
                       torch.nn.functional.silu(g2) * u2)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,sw", [(1, 4096, 6144, 32), (4, 4096, 1024, 16), (8, 2048, 28672, 64),
                                      (1, 14336, 4096, 16), (8, 4096, 6144, 32), (3, 8192, 512, 64)])
def test_rmsnorm_prologue_is_the_two_step_composition(M, K, N, sw):
    _, _, _, Xd, _, sm = strip_case(M, K, N, 128, sw, seed=5)
    w = (torch.rand(K, generator=torch.Generator().manual_seed(K)) + 0.5).half().cuda()
    fused = ng.rmsnorm_matmul(Xd, w, sm, 1e-5)
    # the one-launch form directly (rmsnorm_matmul composes from M = 4)
    direct = ops._strip_gemv(Xd, sm, 0, None, N, (w, 1e-5))
    from nibblegemm_amd.glue import rmsnorm  # noqa: PLC0415

    two_step = ng.matmul(rmsnorm(Xd, w, 1e-5), sm)
    assert torch.equal(fused, two_step)
    assert torch.equal(direct, two_step)


@pytest.mark.gpu
def test_graph_replay_repeats_eager_bits():
    _, _, _, Xd, _, sm = strip_case(1, 14336, 4096, 128, seed=3)
    eager = ng.matmul(Xd, sm)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ng.matmul(Xd, sm)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ng.matmul(Xd, sm)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ng.matmul(Xd, sm)  # eager work between replays


@pytest.mark.gpu
def test_overrides_are_refused():
    _, _, _, Xd, _, sm = strip_case(1, 256, 64, 128, seed=0)
    with pytest.raises(ValueError, match="no splits"):
        ng.matmul(Xd, sm, splits=2)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("M", [9, 16, 17, 24, 32, 33, 64, 128, 129, 512, 2048])
def test_batches_above_8_have_the_packed_bits(M, K, N):
    """From 9 rows a strip-major weight runs the packed weight's plans and
    kernels (streaming, 64-row tiles with a K split, 128 / 256-row tiles),
    reading the strip-major layout: the outputs are the packed call's bits,
    and so as close to the oracle as those (tests/test_gemm.py)."""
    X, packed, scales, Xd, qw, sm = strip_case(M, K, N, 128, seed=M + K)
    got = ng.matmul(Xd, sm)
    assert torch.equal(got, ng.matmul(Xd, qw))
    if M > 128:
        assert torch.equal(ng.gemm(Xd, sm, version=7), ng.gemm(Xd, qw, version=7))
    if M in (17, 129):
        rows = [0, M // 2, M - 1]
        ref = O.reference_matmul(np.ascontiguousarray(X[rows]), packed, scales, K, 128)
        assert rms_err(host(got[rows]), ref.astype(np.float32)) <= RMS_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,g,sw", [(9, 1024, 448, 128, 16), (40, 2048, 512, 64, 32),
                                        (200, 4096, 1024, 128, 16), (100, 1024, 4096, 64, 64),
                                        (1000, 4096, 4096, 128, 32), (16, 4096, 28672, 128, 64),
                                        (24, 4096, 28672, 128, 64), (32, 4096, 28672, 128, 32)])
def test_every_width_above_8_rows_has_the_packed_bits(M, K, N, g, sw):
    """Every strip width from 9 rows: the packed weight's bits, with and
    without the bias epilogue (4096 x 28672 at 24 and 32 rows takes strip
    pairs in the batch kernel)."""
    _, _, _, Xd, qw, sm = strip_case(M, K, N, g, sw, seed=sw + M)
    assert torch.equal(ng.matmul(Xd, sm), ng.matmul(Xd, qw))
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(2)) * 0.3).half().cuda()
    assert torch.equal(ng.matmul_bias(Xd, sm, bias), ng.matmul(Xd, qw) + bias)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,g,sw", [(4096, 14336, 128, 64), (14336, 4096, 128, 16),
                                      (1024, 448, 64, 32), (256, 96, 128, 32)])
@pytest.mark.parametrize("fast", [True, False])
def test_dequant_of_strip_major_weights_is_the_packed_dequant(K, N, g, sw, fast):
    _, _, _, _, qw, sm = strip_case(1, K, N, g, sw, seed=K + N)
    a = ng.dequant(sm, fast=fast)
    assert a.shape == (K, N)
    assert torch.equal(a.view(torch.int16), ng.dequant(qw, fast=fast).view(torch.int16))


def test_strip_major_round_trip_on_the_host():
    _, packed, scales = O.synthetic_case(1, 256, 96, 128, 3)
    qw = quant.QuantizedWeight(torch.from_numpy(packed.view(np.int32)),
                               torch.from_numpy(scales.view(np.float16)), 128, 256, 96)
    for sw in (16, 32):
        back = quant.from_strip_major(quant.strip_major(qw, sw))
        assert torch.equal(back.qweight, qw.qweight) and torch.equal(back.scales, qw.scales)


@pytest.mark.gpu
def test_quantlinear_keeps_one_strip_major_copy():
    """prepare_decode converts the weight in place: one copy, read by every
    batch size; the state dict stays the reference's packed format both
    ways."""
    torch.manual_seed(1)
    lin = torch.nn.Linear(1024, 448).half().cuda()
    ql = ng.QuantLinear.from_linear(lin)
    x = torch.randn(3, 1024, device="cuda").half()
    big = torch.randn(40, 1024, device="cuda").half()
    packed = {k: v.clone() for k, v in ql.state_dict().items()}
    before, before_big = ql(x), ql(big)
    assert ql.prepare_decode() is ql
    sw = ng.strip_major_cols(1024, 448, 128)
    assert ql.strip_cols == sw and tuple(ql.qweight.shape) == (448 // sw, 128, sw)
    assert len(list(ql.buffers())) == 3  # qweight, scales, bias: one copy of the weight
    sd = ql.state_dict()
    assert set(sd) == {"qweight", "scales", "bias"}
    assert all(torch.equal(sd[k], packed[k]) for k in sd)
    sm = ng.StripMajorWeight(ql.qweight, ql.scales, 128, 1024, 448, sw)
    assert torch.equal(ql(x), ng.matmul(x, sm) + ql.bias)
    assert rms_err(host(ql(x)), host(before)) <= 5e-3
    assert torch.equal(ql(big), before_big)  # above 8 rows: the packed weight's bits
    # a packed state dict loads into the strip-major module
    other = ng.QuantLinear.from_linear(torch.nn.Linear(1024, 448).half().cuda())
    ql.load_state_dict(other.state_dict())
    assert torch.equal(ql.state_dict()["qweight"], other.state_dict()["qweight"])
    other.prepare_decode(sw)
    assert torch.equal(ql.qweight, other.qweight) and torch.equal(ql(x), other(x))
    ql.release_decode()
    assert ql.strip_cols == 0 and tuple(ql.qweight.shape) == (128, 448)
    assert torch.equal(ql.qweight, other.state_dict()["qweight"])
    assert torch.equal(ql(x), ng.matmul_bias(x, ql._qw(), ql.bias))
