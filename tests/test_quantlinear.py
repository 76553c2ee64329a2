"""``QuantLinear`` as the drop-in for ``nn.Linear`` (reference
python/nibblegemm/ops.py:107-135), checked against the C oracle.

* ``from_linear`` must produce the oracle's RTN codes and scales of the
  transposed weight: bit for bit for a host layer, and up to the GPU's
  reciprocal rounding of the scalar division for a GPU layer -- a
  transposition or quantisation slip changes nearly every code.
* ``forward`` must match the oracle's dequantize-then-fp32-matmul of those
  codes (plus the bias, added in fp16 as the reference's module does) within
  the north-star bound ``max|y - ref| <= 1e-2 * rms(ref)``, through every
  kernel the batch size reaches: the strip GEMV (M <= 8), the streaming kernel
  (M <= 128) and the MFMA tile kernel (larger M).
* The layer's shape handling, dtypes, devices and state dict follow the
  reference module.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from cases import host, rms_err

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-2
FEATURES = [(384, 200), (1024, 96)]  # (in = K, out = N): K % 128 == 0, N % 4 == 0


def linear_layer(in_f: int, out_f: int, bias: bool, seed: int, device="cuda") -> torch.nn.Linear:
    gen = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(in_f, out_f, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(out_f, in_f, generator=gen) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(out_f, generator=gen) * 0.1)
    return lin.half().to(device)


def oracle_forward(oracle, x: np.ndarray, ql: ng.QuantLinear) -> np.ndarray:
    """The reference module's arithmetic on the host: fp16(X @ dequant), then
    the fp16 bias add."""
    packed = ql.qweight.cpu().numpy()
    scales = ql.scales.cpu().numpy()
    y = oracle.reference_matmul(x, packed, scales, ql.K, ql.group_size)
    if ql.bias is not None:
        y = (y.astype(np.float32) + ql.bias.cpu().numpy().astype(np.float32)).astype(np.float16)
    return y.astype(np.float32)


def oracle_codes(oracle, lin: torch.nn.Linear, group_size: int):
    codes, _, s16 = oracle.quantize_rtn(lin.weight.detach().float().t().cpu().numpy(), group_size)
    return oracle.pack_nibbles(codes), s16


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("in_f,out_f", FEATURES)
def test_from_linear_is_the_oracle_quantisation(oracle, in_f, out_f, group_size):
    """A host layer quantises on the host: the oracle's codes and scales of
    the transposed weight, bit for bit."""
    lin = linear_layer(in_f, out_f, bias=True, seed=in_f + out_f, device="cpu")
    ql = ng.QuantLinear.from_linear(lin, group_size=group_size)
    assert (ql.K, ql.N, ql.group_size) == (in_f, out_f, group_size)
    assert ql.qweight.dtype == torch.int32 and tuple(ql.qweight.shape) == (in_f // 8, out_f)
    assert ql.scales.dtype == torch.float16 and tuple(ql.scales.shape) == (in_f // group_size, out_f)
    packed, s16 = oracle_codes(oracle, lin, group_size)
    assert np.array_equal(ql.qweight.numpy(), packed)
    assert np.array_equal(ql.scales.numpy().view(np.uint16), s16.view(np.uint16))
    assert torch.equal(ql.bias, lin.bias)


@pytest.mark.parametrize("in_f,out_f", FEATURES)
def test_from_linear_on_the_gpu(oracle, in_f, out_f):
    """A GPU layer quantises on the GPU with the reference's operations; its
    max-abs scale divides by the scalar 7, which a GPU applies as a multiply
    by the reciprocal, so a rare scale sits one fp32 ulp from the oracle's
    true division (and a code on a rounding tie with it).  Everything else is
    the oracle's quantisation of the transposed weight (a transposed or
    regrouped weight would change nearly every code)."""
    lin = linear_layer(in_f, out_f, bias=False, seed=9)
    ql = ng.QuantLinear.from_linear(lin)
    assert ql.qweight.is_cuda and ql.scales.is_cuda
    packed, s16 = oracle_codes(oracle, lin, 128)
    got = ng.unpack_nibbles(ql.qweight.cpu().numpy(), in_f)
    want = ng.unpack_nibbles(packed, in_f)
    assert (got != want).mean() < 1e-3
    ds = np.abs(ql.scales.cpu().numpy().view(np.uint16).astype(np.int32) - s16.view(np.uint16))
    assert ds.max() <= 1 and (ds != 0).mean() < 1e-2


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M", [1, 3, 8, 24, 128, 200])
@pytest.mark.parametrize("in_f,out_f", FEATURES)
def test_forward_matches_the_oracle(oracle, in_f, out_f, M, bias):
    lin = linear_layer(in_f, out_f, bias, seed=7 * M + in_f)
    ql = ng.QuantLinear.from_linear(lin)
    gen = torch.Generator().manual_seed(M)
    x = torch.randn(M, in_f, generator=gen).half()
    y = ql(x.cuda())
    assert y.shape == (M, out_f) and y.dtype == torch.float16
    assert rms_err(host(y), oracle_forward(oracle, x.numpy(), ql)) <= RMS_TOL


@pytest.mark.parametrize("lead", [(2, 3), (1, 1, 5), (4,), (6, 33)])
def test_leading_dimensions_are_kept(lead):
    ql = ng.QuantLinear.from_linear(linear_layer(384, 200, bias=True, seed=1))
    x = torch.randn(*lead, 384, device="cuda").half()
    y = ql(x)
    assert y.shape == (*lead, 200)
    assert torch.equal(y.reshape(-1, 200), ql(x.reshape(-1, 384)))


@pytest.mark.parametrize("M", [1, 16, 160])
def test_fp16_bias_has_the_bits_of_a_separate_add(M):
    """The fused bias epilogue (M <= 128) and the two-op path give
    fp16(fp16(X W) + b) exactly."""
    ql = ng.QuantLinear.from_linear(linear_layer(1024, 96, bias=True, seed=2))
    x = torch.randn(M, 1024, device="cuda").half()
    qw = ng.QuantizedWeight(ql.qweight, ql.scales, ql.group_size, ql.K, ql.N)
    assert torch.equal(ql(x), ng.matmul(x, qw) + ql.bias)


def test_fp32_bias_promotes_like_the_reference():
    ql = ng.QuantLinear.from_linear(linear_layer(384, 200, bias=True, seed=3))
    ql.bias = ql.bias.float()
    x = torch.randn(5, 384, device="cuda").half()
    y = ql(x)
    qw = ng.QuantizedWeight(ql.qweight, ql.scales, ql.group_size, ql.K, ql.N)
    assert y.dtype == torch.float32
    assert torch.equal(y, ng.matmul(x, qw) + ql.bias)


def test_without_bias_forward_is_matmul():
    ql = ng.QuantLinear.from_linear(linear_layer(384, 200, bias=False, seed=4))
    assert ql.bias is None and set(ql.state_dict()) == {"qweight", "scales"}
    x = torch.randn(7, 384, device="cuda").half()
    qw = ng.QuantizedWeight(ql.qweight, ql.scales, ql.group_size, ql.K, ql.N)
    assert torch.equal(ql(x), ng.matmul(x, qw))


def test_state_dict_reloads_into_a_fresh_module():
    src = ng.QuantLinear.from_linear(linear_layer(1024, 96, bias=True, seed=5), group_size=64)
    sd = src.state_dict()
    assert set(sd) == {"qweight", "scales", "bias"}
    blank = ng.QuantizedWeight(torch.zeros_like(src.qweight), torch.zeros_like(src.scales), 64,
                               1024, 96)
    dst = ng.QuantLinear(blank, torch.zeros_like(src.bias))
    dst.load_state_dict(sd)
    x = torch.randn(3, 1024, device="cuda").half()
    assert torch.equal(dst(x), src(x))


def test_from_linear_keeps_the_layer_device():
    lin = torch.nn.Linear(256, 64).half()  # on the host
    ql = ng.QuantLinear.from_linear(lin)
    assert not ql.qweight.is_cuda and not ql.scales.is_cuda and not ql.bias.is_cuda
