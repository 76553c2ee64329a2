"""The fused output epilogues of the streaming kernel (nibble_matmul_w4a16_fused).

Both epilogues are defined as the unfused fp16 ops they replace, so the test
is bit equality with those ops run separately on the GPU:
  * bias:   matmul(X, W) + bias               (the reference QuantLinear, ops.py:131-135)
  * swiglu: silu(G) * U, G | U the halves of X [W_gate | W_up]  (the fp16 torch composition)
and, for SwiGLU, the north-star tolerance against an fp32 evaluation of the
same MLP input from the oracle's products.
"""
from __future__ import annotations

import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import ops
from nibblegemm_amd.quant import split_swiglu
from cases import host, oracle_y, synthetic, quantized

pytestmark = pytest.mark.gpu

SHAPES = [(1, 4096, 1024, 128), (4, 512, 260, 64), (8, 14336, 512, 128), (16, 1024, 4100, 128),
          (12, 4096, 14336, 128), (100, 2048, 640, 64), (128, 8192, 384, 128),
          (64, 14336, 4096, 128), (17, 14336, 4096, 128), (24, 4096, 1028, 64), (32, 4096, 14336, 128),
          (24, 4096, 28672, 128)]


@pytest.mark.parametrize("M,K,N,g", SHAPES)
def test_bias_epilogue_is_the_separate_add(M, K, N, g):
    _, _, _, Xd, qw = synthetic(M, K, N, g, seed=M + K + N)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(N)) * 0.5).half().cuda()
    fused = ng.matmul_bias(Xd, qw, bias)
    separate = ng.matmul(Xd, qw) + bias
    assert fused.dtype == torch.float16 and fused.shape == (M, N)
    assert torch.equal(fused, separate)


SWIGLU = [(1, 4096, 1024, 128), (8, 14336, 512, 128), (16, 4096, 14336, 128), (33, 1024, 320, 64),
          (128, 2048, 96, 128), (48, 4096, 14336, 128), (24, 4096, 4096, 128), (32, 2048, 640, 64),
          (20, 4096, 14336, 128)]


@pytest.mark.parametrize("M,K,Nh,g", SWIGLU)
def test_swiglu_epilogue_is_the_fp16_composition(M, K, Nh, g):
    Xg, pg, sg, Xd, gate = quantized(M, K, Nh, g, seed=1)
    _, pu, su, _, up = quantized(M, K, Nh, g, seed=2)
    qw = ng.interleave_swiglu(gate, up)
    fused = ng.matmul_swiglu(Xd, qw)
    assert fused.shape == (M, Nh)
    # The fused output is the fp16 SwiGLU of the gate|up product's halves.
    yg, yu = split_swiglu(ng.matmul(Xd, qw))
    assert torch.equal(fused, torch.nn.functional.silu(yg) * yu)
    if M <= 16 and ng.extension().gemm_streams(M, K, 2 * Nh, g):
        # Up to 16 rows the streaming plan splits K by K alone, so the gate
        # and up products on their own sum in the same order.  (Larger
        # batches split K by the strip or tile count too: there the
        # products of N / 2 columns may sum in another order.)
        composed = torch.nn.functional.silu(ng.matmul(Xd, gate)) * ng.matmul(Xd, up)
        assert torch.equal(fused, composed)
    # against fp32 arithmetic on the oracle's products of the same inputs:
    # 1e-2 of the RMS, plus, per element, the fp16 rounding of its own value
    # (the product's heavy tail puts its largest outputs ~30 RMS out, where
    # one fp16 ulp alone is ~1.5e-2 RMS)
    yg = torch.from_numpy(oracle_y(Xg, pg, sg, K, g)).float()
    yu = torch.from_numpy(oracle_y(Xg, pu, su, K, g)).float()
    ref = torch.nn.functional.silu(yg) * yu
    rms = ref.pow(2).mean().sqrt()
    diff = (torch.from_numpy(host(fused)).float() - ref).abs()
    assert bool((diff <= 1e-2 * rms + 2.0 ** -10 * ref.abs()).all())


def test_swiglu_above_the_fused_batch_limit_composes():
    M, K, Nh, g = 200, 512, 128, 128
    _, _, _, Xd, gate = quantized(M, K, Nh, g, seed=3)
    _, _, _, _, up = quantized(M, K, Nh, g, seed=4)
    y = ng.matmul_swiglu(Xd, ng.interleave_swiglu(gate, up))
    composed = torch.nn.functional.silu(ng.matmul(Xd, gate)) * ng.matmul(Xd, up)
    assert torch.equal(y, composed)


def test_quantlinear_bias_fused_and_promoting():
    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 256, bias=True).half().cuda()
    ql = ng.QuantLinear.from_linear(lin, group_size=128)
    x = torch.randn(2, 3, 512, device="cuda").half()
    y = ql(x)
    expect = (ng.matmul(x.reshape(-1, 512), ql._qw()) + ql.bias).reshape(2, 3, 256)
    assert torch.equal(y, expect)
    # an fp32 bias promotes the result, as the reference's fp16 + fp32 add does
    ql32 = ng.QuantLinear(ql._qw(), ql.bias.float())
    y32 = ql32(x)
    assert y32.dtype == torch.float32
    assert torch.equal(y32, ng.matmul(x.reshape(-1, 512), ql._qw()).reshape(2, 3, 256) + ql32.bias)


def test_fused_calls_replay_in_a_graph():
    """Split-K counters of the fused launch are reset in-kernel: captured calls
    replay correctly, with eager work between replays."""
    M, K, N, g = 4, 14336, 512, 128
    _, _, _, Xd, qw = synthetic(M, K, N, g, seed=5)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(5)).half().cuda()
    ref = ng.matmul_bias(Xd, qw, bias)
    assert ops._fused_workspace(ops._bind(), Xd.device, ops._stream(Xd.device), M, K, N, g)[0] is not None
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ng.matmul_bias(Xd, qw, bias)  # warm the capture-side workspace cache
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ng.matmul_bias(Xd, qw, bias)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        ng.matmul(Xd, qw)  # eager work between replays
        torch.cuda.synchronize()


def test_fused_plans_sharing_a_workspace():
    """The fused entry sizes its workspace for the larger of its two plans and
    lays it out that way (counters, then partials), so plans whose own
    counter regions differ can share the buffer the package keys by the
    reported counter size: a 64-row bias call (64 strips split 4 ways) and
    then a 24-row SwiGLU (128 strips split 2 ways) both report 512 counter
    bytes; the second must not read the first's partials as counters."""
    ext = ng.extension()
    assert ext.matmul_fused_workspace_bytes(64, 14336, 4096, 128, None)[1] == \
        ext.matmul_fused_workspace_bytes(24, 4096, 8192, 128, None)[1]
    _, _, _, X1, w1 = synthetic(64, 14336, 4096, 128, seed=5)
    bias = (torch.randn(4096, generator=torch.Generator().manual_seed(4)) * 0.5).half().cuda()
    assert torch.equal(ng.matmul_bias(X1, w1, bias), ng.matmul(X1, w1) + bias)
    _, _, _, X2, gate = quantized(24, 4096, 4096, 128, seed=1)
    _, _, _, _, up = quantized(24, 4096, 4096, 128, seed=2)
    qw = ng.interleave_swiglu(gate, up)
    for _ in range(3):
        fused = ng.matmul_swiglu(X2, qw)
        yg, yu = split_swiglu(ng.matmul(X2, qw))
        assert torch.equal(fused, torch.nn.functional.silu(yg) * yu)
        assert torch.equal(ng.matmul_bias(X1, w1, bias), ng.matmul(X1, w1) + bias)
