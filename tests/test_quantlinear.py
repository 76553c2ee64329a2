"""QuantLinear as a drop-in nn.Linear replacement (reference
tests/test_quantlinear.py intents): the kernel's error against exact math on
the same INT4 weights must be small next to the error quantisation opens."""
from __future__ import annotations

import pytest
import torch

import nibblegemm_amd as ng
from cases import rel_err

pytestmark = pytest.mark.gpu

IN, OUT = 256, 128
REL_TOL = 5e-2


def make_layer(bias: bool, group_size: int = 128, seed: int = 0):
    torch.manual_seed(seed)
    linear = torch.nn.Linear(IN, OUT, bias=bias).cuda().half()
    return linear, ng.QuantLinear.from_linear(linear, group_size=group_size)


def quantized_weight(ql: ng.QuantLinear) -> ng.QuantizedWeight:
    return ng.QuantizedWeight(ql.qweight, ql.scales, ql.group_size, ql.K, ql.N)


def np_(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M", [1, 8, 64])
@pytest.mark.parametrize("group_size", [64, 128])
def test_error_belongs_to_quantisation_not_to_the_kernel(bias, M, group_size):
    linear, ql = make_layer(bias, group_size)
    x = torch.randn(M, IN, device="cuda", dtype=torch.float16)
    y = ql(x)
    assert y.shape == (M, OUT) and y.dtype == torch.float16

    exact_int4 = ng.reference_matmul(x, quantized_weight(ql))
    if bias:
        exact_int4 = exact_int4 + ql.bias
    exact_fp16 = linear(x)
    kernel_err = (y.float() - exact_int4.float()).abs().mean().item()
    quant_err = (exact_int4.float() - exact_fp16.float()).abs().mean().item()
    assert quant_err > 0.0
    assert kernel_err < 0.25 * quant_err
    assert rel_err(np_(y), np_(exact_int4)) < REL_TOL


@pytest.mark.parametrize("shape", [(1, 4, IN), (2, 8, IN), (3, 1, IN), (2, 64, IN)])
def test_3d_input_is_flattened_and_restored(shape):
    _, ql = make_layer(bias=True, seed=1)
    x = torch.randn(*shape, device="cuda", dtype=torch.float16)
    y = ql(x)
    assert y.shape == (*shape[:-1], OUT)
    flat = ng.reference_matmul(x.reshape(-1, IN), quantized_weight(ql)) + ql.bias
    assert rel_err(np_(y.reshape(-1, OUT)), np_(flat)) < REL_TOL


def test_bias_is_added_exactly():
    _, ql = make_layer(bias=True, seed=2)
    x = torch.randn(4, IN, device="cuda", dtype=torch.float16)
    assert torch.equal(ql(x), ng.matmul(x, quantized_weight(ql)) + ql.bias)


def test_no_bias_is_a_plain_matmul():
    _, ql = make_layer(bias=False, seed=3)
    assert ql.bias is None
    x = torch.randn(4, IN, device="cuda", dtype=torch.float16)
    assert torch.equal(ql(x), ng.matmul(x, quantized_weight(ql)))


def test_from_linear_transposes_the_weight():
    linear, ql = make_layer(bias=False, seed=4)
    assert (ql.K, ql.N) == (IN, OUT)
    approx = ng.dequantize(quantized_weight(ql)).float()
    truth = linear.weight.data.t().float().cpu()
    assert approx.shape == truth.shape
    assert (approx - truth).abs().mean() < 0.25 * truth.abs().mean()


def test_state_dict_round_trip():
    _, ql = make_layer(bias=True, seed=5)
    sd = ql.state_dict()
    assert set(sd) == {"qweight", "scales", "bias"}
    ql2 = ng.QuantLinear(ng.QuantizedWeight(torch.empty_like(ql.qweight), torch.empty_like(ql.scales),
                                            ql.group_size, ql.K, ql.N), torch.empty_like(ql.bias))
    ql2.load_state_dict(sd)
    x = torch.randn(3, IN, device="cuda", dtype=torch.float16)
    assert torch.equal(ql(x), ql2(x))
