"""The config-5 decode-step driver and the device quantiser it relies on."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import decode_step as D


def test_tensor_parallel_shares():
    """One GPU's share of a tp-way split: q, k, v, gate, up by output columns,
    o and down by input rows in whole quant groups; splits that would cut a
    16-column SwiGLU block or a quant group are refused."""
    full = D.projection_shapes()
    assert full == D.projection_shapes(tp=1)
    eight = D.projection_shapes(tp=8)
    assert eight == {"q": (4096, 512), "k": (4096, 128), "v": (4096, 128), "o": (512, 4096),
                     "gate": (4096, 1792), "up": (4096, 1792), "down": (1792, 4096)}
    for tp in (2, 4, 8, 16):
        share = D.projection_shapes(tp=tp)
        for name, (K, N) in full.items():
            k, n = share[name]
            assert (k * tp, n) == (K, N) if name in ("o", "down") else (k, n * tp) == (K, N)
    with pytest.raises(ValueError):
        D.projection_shapes(tp=3)       # 14336 / 3
    with pytest.raises(ValueError):
        D.projection_shapes(tp=32)      # 14336 / 32 = 448 rows: not whole groups of 128
    with pytest.raises(ValueError):
        D.projection_shapes(tp=0)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,g", [(4096, 1024, 128), (512, 264, 64), (14336, 128, 128)])
def test_quantize_device_is_bit_identical_to_the_oracle(oracle, K, N, g):
    gen = torch.Generator().manual_seed(K + N)
    W = torch.randn(K, N, generator=gen) * 0.02
    W[:g, 0] = 0.0                                   # zero group
    W[:g, 1] = torch.arange(g, dtype=torch.float32)  # exact ties after scaling
    qw = ng.quantize_device(W.cuda(), group_size=g)
    assert qw.qweight.is_cuda and qw.scales.is_cuda
    qu, _, s16 = oracle.quantize_rtn(W.numpy(), g)
    assert np.array_equal(qw.qweight.cpu().numpy(), oracle.pack_nibbles(qu))
    assert np.array_equal(qw.scales.cpu().numpy().view(np.uint16), s16.view(np.uint16))


@pytest.mark.gpu
def test_concatenated_gemv_equals_the_separate_ones():
    """q|k|v and gate|up fusion: one launch over 64-column-aligned parts gives
    the same bits per column as separate launches."""
    gen = torch.Generator(device="cuda").manual_seed(3)
    parts = [ng.quantize_device(torch.randn(4096, n, generator=gen, device="cuda") * 0.02)
             for n in (4096, 1024, 1024)]
    x = torch.randn(1, 4096, generator=gen, device="cuda").half()
    fused = ng.matmul(x, ng.concat_columns(*parts))
    sep = torch.cat([ng.matmul(x, p) for p in parts], dim=1)
    assert torch.equal(fused, sep)


@pytest.mark.gpu
def test_decode_step_runs_and_counts_launches():
    cfg = {"hidden": 512, "kv": 128, "intermediate": 1024, "layers": 2}
    layers = D.build_layers(2, cfg=cfg)
    step = D.DecodeStep(layers)
    assert step.launches == 14
    step()
    fused = D.DecodeStep([D.fuse(layer) for layer in layers])
    assert fused.launches == 8
    fused()
    sw = D.DecodeStep([D.fuse(layer, swiglu=True) for layer in layers])
    assert sw.launches == 8
    sw()
    torch.cuda.synchronize()
    # the SwiGLU launch writes silu(gate) * up, the input width of down
    layer = layers[0]
    x = torch.randn(1, 512, device="cuda").half()
    h = ng.matmul_swiglu(x, D.fuse(layer, swiglu=True)["gate_up_swiglu"])
    assert h.shape == (1, 1024)
    assert torch.equal(h, torch.nn.functional.silu(ng.matmul(x, layer["gate"])) * ng.matmul(x, layer["up"]))
    nbytes = D.weight_bytes(layers)
    shapes = D.projection_shapes(cfg)
    assert nbytes == 2 * sum(k * n // 2 + (k // 128) * n * 2 for k, n in shapes.values())


# ---------------------------------------------------------------------------
# The config-5 step at its real shapes (2 distinct Llama-3-8B layers)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def layers_8b():
    return D.build_layers(2, seed=21)


def _replays_match(run, between, replays: int = 3):
    """``run()`` captured in a HIP graph: every replay, with eager work and
    synchronisation in between, reproduces the eager outputs bit for bit."""
    eager = [t.clone() for t in run()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = run()
    torch.cuda.synchronize()
    for _ in range(replays):
        for t in outs:
            t.zero_()
        between()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            assert torch.equal(got, want)
    return eager


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["projections", "fused", "fused_swiglu"])
def test_full_size_step_graph_replays_equal_eager(layers_8b, variant):
    layers = {"projections": layers_8b,
              "fused": [D.fuse(layer) for layer in layers_8b],
              "fused_swiglu": [D.fuse(layer, swiglu=True) for layer in layers_8b]}[variant]
    step = D.DecodeStep(layers)
    assert step.launches == {"projections": 14, "fused": 8, "fused_swiglu": 8}[variant]
    other = D.DecodeStep(layers_8b[:1], seed=5)
    _replays_match(step.outputs, other)


@pytest.mark.gpu
def test_full_size_glue_step_graph_replays_equal_eager(layers_8b):
    layers = [D.fuse(layer, swiglu=True) for layer in layers_8b]
    step = D.GlueDecodeStep(layers, pos=300, max_seq=320)
    other = D.DecodeStep(layers_8b[:1], seed=6)
    _replays_match(lambda: [step()], other)


@pytest.mark.gpu
def test_full_size_fused_launches_equal_the_separate_ones(layers_8b):
    """Each fused launch computes its columns with the separate launches'
    plan, so q|k|v and gate|up give the separate outputs' bits, and the SwiGLU
    epilogue the bits of silu(gate) * up in fp16."""
    layer = layers_8b[1]
    x = torch.randn(1, 4096, device="cuda").half()
    sep = {name: ng.matmul(x, layer[name]) for name in ("q", "k", "v", "gate", "up")}
    fused = D.fuse(layer)
    assert torch.equal(ng.matmul(x, fused["qkv"]), torch.cat([sep["q"], sep["k"], sep["v"]], 1))
    assert torch.equal(ng.matmul(x, fused["gate_up"]), torch.cat([sep["gate"], sep["up"]], 1))
    h = ng.matmul_swiglu(x, D.fuse(layer, swiglu=True)["gate_up_swiglu"])
    assert torch.equal(h, torch.nn.functional.silu(sep["gate"]) * sep["up"])


@pytest.mark.gpu
def test_full_size_projections_match_the_oracle(oracle, layers_8b):
    """Layer 0's seven projections at M = 1 against the oracle's dequantize +
    fp32 matmul, within the north-star bound."""
    step = D.DecodeStep(layers_8b[:1])
    outs = step.outputs()
    for (x, qw, _), y in zip(step.calls, outs):
        ref = oracle.reference_matmul(x.cpu().numpy(), qw.qweight.cpu().numpy(),
                                      qw.scales.cpu().numpy(), qw.K, qw.group_size)
        ref = ref.astype(np.float64)
        err = float(np.abs(y.float().cpu().numpy() - ref).max() / np.sqrt(np.mean(ref ** 2)))
        assert err <= 1e-2, (qw.K, qw.N, err)


@pytest.mark.gpu
@pytest.mark.parametrize("tp", [2, 8])
def test_tensor_parallel_share_projections_match_the_oracle(oracle, tp):
    """One layer at one GPU's share of a tp-way split, each projection on
    packed and strip-major weights, q|k|v and gate|up fused too, against the
    oracle at M = 1."""
    layers = D.build_layers(1, seed=30 + tp, tp=tp)
    fused = [D.fuse(layers[0])]
    for packed in (layers, fused):
        steps = (D.DecodeStep(packed), D.DecodeStep(D.strips(packed)))
        outs = [step.outputs() for step in steps]
        for n, (x, qw, _) in enumerate(steps[0].calls):
            ref = oracle.reference_matmul(x.cpu().numpy(), qw.qweight.cpu().numpy(),
                                          qw.scales.cpu().numpy(), qw.K, qw.group_size)
            ref = ref.astype(np.float64)
            rms = np.sqrt(np.mean(ref ** 2))
            for y in (outs[0][n], outs[1][n]):
                err = float(np.abs(y.float().cpu().numpy() - ref).max() / rms)
                assert err <= 1e-2, (tp, qw.K, qw.N, err)
