"""Persistent decode chains (``nibble_chain_*``, ``nibblegemm_amd.chain``).

* CPU: every rejection of ``nibble_chain_create`` happens in host code before
  any HIP call -- bad shapes, widths and epilogues, ``after`` links that do
  not point back, and stages that read or overwrite another stage's output
  without an ``after`` path ordering them.
* GPU: a chain's outputs have the bits of the per-projection strip-major
  launches (``matmul`` / ``matmul_bias`` / ``matmul_swiglu``) on the same
  weights, for independent stages of every strip width and epilogue, for
  batches of up to 8 rows, and for the dependent data flow of two full-size
  Llama-3-8B layers (each stage reading the previous one's output), also
  replayed from a HIP graph; the strip launches themselves are checked
  against the C oracle in tests/test_strip_major.py.  Repeated runs repeat
  their bits (the counters return to zero), and the wait flag stays clear.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import _native, chain as C, decode_step as D, quant
from cases import host, oracle_y, rms_err, synthetic

OK, INVALID = 0, 1
A = 1 << 20  # aligned fake device addresses, never dereferenced on the CPU tier
W0, S0 = 1 << 40, 1 << 41  # fake weight addresses, far from the activations


def _pack(X=A, Wt=W0, St=S0, Y=A * 4, bias=0, K=4096, N=4096, g=128, sw=16, ep=0, after=-1,
          layout=0):
    return struct.pack("<5Q7q", X, Wt, St, Y, bias, K, N, g, sw, ep, after, layout)


def _create(stages, M=1):
    ext = _native.binding()
    rc, handle = ext.chain_create(b"".join(stages), len(stages), M, None)
    if rc == OK:
        ext.chain_destroy(handle)
    return rc, ext.last_error()


# ---------------------------------------------------------------- CPU tier

@pytest.mark.parametrize("stages,M,needle", [
    ([_pack()], 0, "batches of 1..8"),
    ([_pack()], 9, "batches of 1..8"),
    ([_pack(g=96)], 1, "group_size must be 64 or 128"),
    ([_pack(), _pack(Y=A * 5, g=64, sw=32)], 1, "share group_size"),
    ([_pack(sw=24)], 1, "no strip-major plan"),
    ([_pack(N=4016, sw=32)], 1, "no strip-major plan"),
    ([_pack(K=4000)], 1, "bad K"),
    ([_pack(ep=3)], 1, "epilogue must be"),
    ([_pack(ep=2, sw=16, N=4096)], 1, "swiglu needs strips of at least 32"),
    ([_pack(ep=1)], 1, "null bias"),
    ([_pack(X=A + 8)], 1, "alignment"),
    ([_pack(after=0)], 1, "earlier stage"),
    ([_pack(), _pack(Y=A * 5, after=1)], 1, "earlier stage"),
    ([_pack(X=A * 4)], 1, "overlaps its own inputs"),
    # stage 1 reads stage 0's output without waiting for it
    ([_pack(), _pack(X=A * 4, Y=A * 5)], 1, "without waiting"),
    # stage 1 overwrites what stage 0 reads
    ([_pack(), _pack(X=A * 6, Y=A)], 1, "overwrites what stage 0 reads"),
    # two stages write the same output unordered
    ([_pack(), _pack(X=A * 6)], 1, "without waiting"),
    # a stage writes weights
    ([_pack(), _pack(X=A * 6, Y=W0 + 64, after=0)], 1, "weights"),
    ([_pack(Y=S0 + 1024)], 1, "weights"),
    ([_pack(layout=2)], 1, "layout must be"),
    ([_pack(layout=1, N=4000, sw=64)], 1, "no strip-major plan"),
])
def test_create_rejections(stages, M, needle):
    rc, msg = _create(stages, M)
    assert rc == INVALID and needle in msg, (rc, msg)


def test_create_rejects_bad_bytes():
    ext = _native.binding()
    with pytest.raises(ValueError, match="need"):
        ext.chain_create(_pack()[:-8], 1, 1, None)
    with pytest.raises(TypeError):
        ext.chain_create("not bytes", 1, 1, None)


def test_ordered_hazards_pass_validation():
    """Reads and writes ordered through a chain of ``after`` links (directly
    or transitively) are accepted up to the first HIP call, which fails on a
    machine without a GPU with a HIP error instead of a validation error."""
    stages = [_pack(),                                   # 0: X -> Y0
              _pack(X=A * 4, Y=A * 5, after=0),          # 1: reads Y0
              _pack(X=A * 5, Y=A * 6, after=1),          # 2: reads Y1
              _pack(X=A * 4, Y=A * 7, after=2),          # 3: reads Y0 (transitively after 0)
              _pack(X=A * 7, Y=A * 4, after=3)]          # 4: overwrites Y0 after its readers
    rc, msg = _create(stages)
    if torch.cuda.is_available():
        assert rc in (OK, 4), msg  # fake pointers: a GPU box reaches the allocation
    else:
        assert rc != INVALID, msg


def test_python_stage_checks():
    X = torch.zeros(1, 256, dtype=torch.float16)
    w = quant.StripMajorWeight(torch.zeros(4, 32, 32, dtype=torch.int32),
                               torch.zeros(4, 2, 32, dtype=torch.float16), 128, 256, 128, 32)
    with pytest.raises(RuntimeError, match="GPU"):
        C.DecodeChain([C.stage(X, w)])
    with pytest.raises(ValueError, match="exclusive"):
        C.stage(X, w, bias=torch.zeros(128, dtype=torch.float16), swiglu=True)
    with pytest.raises(ValueError, match="at least one"):
        C.DecodeChain([])


# ---------------------------------------------------------------- GPU tier

def _run(chain: C.DecodeChain):
    chain.run()
    chain.check()
    return [y.clone() for y in chain.outputs()]


@pytest.mark.parametrize("K,N,g,M,want", [
    (14336, 4096, 128, 1, 32),   # down: 64-column strips of K = 14336 exceed the LDS
    (4096, 4096, 128, 1, 64),    # o (the launches: 16)
    (4096, 1024, 128, 1, 64),    # k, v
    (4096, 6144, 128, 1, 64),    # q|k|v (the launches: 32)
    (4096, 28672, 128, 1, 64),   # gate|up: already the launches' 64
    (4096, 1024, 64, 1, 64),
    (1792, 4096, 128, 1, 64),    # down at one GPU's share of an 8-way split
    (4096, 96, 128, 1, 32),      # 96 columns hold no 64-column strip
    (4096, 16, 128, 1, 16),      # 16 columns hold no 32-column strip
    (14336, 4096, 128, 2, 0),    # two rows of K = 14336 exceed the LDS at any width
    (4096, 4096, 128, 8, 0),
    (4096, 4096, 128, 9, 0),     # chains serve 1..8 rows
    (4096, 40, 128, 1, 0),       # no strip-major layout
])
def test_chain_strip_width(K, N, g, M, want):
    assert C.chain_strip_cols(K, N, g, M) == want


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M", [(14336, 4096, 1), (4096, 4096, 1), (4096, 1024, 2),
                                   (4096, 28672, 1), (14336, 4096, 2), (4096, 4096, 8)])
def test_chain_strip_width_agrees_with_the_plan(K, N, M):
    """A one-stage chain accepts the width the query gives; where the query
    gives 0, the launches' width is rejected for its LDS."""
    gen = torch.Generator().manual_seed(K + N + M)
    codes = torch.randint(0, 16, (K, N), generator=gen, dtype=torch.uint8).numpy()
    scales = (torch.rand((K // 128, N), generator=gen) * 0.01 + 0.001).to(torch.float16)
    qw = quant.QuantizedWeight(torch.from_numpy(quant.pack_nibbles(codes)).cuda(), scales.cuda(),
                               128, K, N)
    X = torch.randn((M, K), generator=gen).to(torch.float16).cuda()
    sw = C.chain_strip_cols(K, N, 128, M)
    if sw:
        sm = ng.to_strip_major(qw, sw)
        chain = C.DecodeChain([C.stage(X, sm)], M=M)
        got = _run(chain)[0]
        assert torch.equal(got, ng.matmul(X, sm))
        chain.close()
    else:
        with pytest.raises(RuntimeError, match="bytes of LDS"):
            C.DecodeChain([C.stage(X, ng.to_strip_major(qw, ng.strip_major_cols(K, N, 128)))], M=M)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 5, 8])
def test_independent_stages_have_the_strip_launch_bits(M):
    """Every strip width (16 / 32 / 64 columns, 8 / 8 / 4 waves), the bias and
    SwiGLU epilogues and long K, as independent stages of one chain."""
    shapes = [(1024, 4096), (4096, 4096), (4096, 6144), (4096, 14336), (14336, 4096),
              (4096, 1024), (2048, 512), (8192, 2048), (1024, 14336), (1024, 512)]
    # The two activation buffers (MT rows of the largest K) must fit LDS
    # beside the weight rings: K up to 14336 / 4096 / 2048 / 1024 for
    # 1 / 2 / 4 / 8-row blocks.
    kmax = {1: 14336, 2: 4096, 4: 2048, 8: 1024}[1 if M == 1 else 2 if M == 2 else 4 if M <= 4 else 8]
    ke = min(kmax, 4096)  # K of the epilogue stages
    stages, want = [], []
    for i, (K, N) in enumerate(shapes):
        if K > kmax:
            continue
        X, packed, scales, Xd, qw = synthetic(M, K, N, 128, seed=i + 10 * M)
        sm = ng.to_strip_major(qw)
        stages.append(C.stage(Xd, sm))
        want.append(ng.matmul(Xd, sm))
        if K == 1024 and N == 4096:
            assert rms_err(host(want[-1]), oracle_y(X, packed, scales, K, 128)) <= 1e-2
    # epilogues
    _, _, _, Xd, qw = synthetic(M, ke, 1024, 128, seed=50)
    sm = ng.to_strip_major(qw)
    bias = (torch.randn(1024, generator=torch.Generator().manual_seed(1)) * 0.3).half().cuda()
    stages.append(C.stage(Xd, sm, bias=bias))
    want.append(ng.matmul_bias(Xd, sm, bias))
    _, _, _, Xd, gate = synthetic(M, ke, 2048, 128, seed=51)
    _, _, _, _, up = synthetic(M, ke, 2048, 128, seed=52)
    for sw in (32, 64):
        smg = ng.to_strip_major(ng.interleave_swiglu(gate, up), sw)
        stages.append(C.stage(Xd, smg, swiglu=True))
        want.append(ng.matmul_swiglu(Xd, smg))
    chain = C.DecodeChain(stages, M=M)
    got = _run(chain)
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), (M, i)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 5])
def test_packed_stages_have_the_strip_major_bits(M):
    """Stages on packed weights (the reference's layout, unconverted) read as
    16-, 32- and 64-column strips, group sizes 128 and 64, the bias and SwiGLU
    epilogues and long K, beside strip-major stages in one chain: every
    output has the bits of the same stage on the strip-major copy at that
    width, which are the strip launch's."""
    kmax = {1: 14336, 2: 4096, 5: 1024}[M]
    cases = [(4096, 4096, 128, 64), (4096, 1024, 128, 32), (1024, 448, 128, 16), (2048, 512, 64, 32),
             (1024, 4096, 64, 64), (14336, 4096, 128, 32), (4096, 6144, 128, 64)]
    stages, want = [], []
    for i, (K, N, g, sw) in enumerate(cases):
        if K > kmax:
            continue
        if g != 128:
            continue  # a chain shares one group size: the group-64 stages go below
        _, _, _, Xd, qw = synthetic(M, K, N, g, seed=70 + i + 10 * M)
        sm = ng.to_strip_major(qw, sw)
        stages.append(C.stage(Xd, qw, strip_cols=sw))
        want.append(ng.matmul(Xd, sm))
        stages.append(C.stage(Xd, sm))  # the same stage on the strip-major copy
        want.append(want[-1])
    ke = min(kmax, 4096)
    _, _, _, Xd, qw = synthetic(M, ke, 1024, 128, seed=80)
    bias = (torch.randn(1024, generator=torch.Generator().manual_seed(3)) * 0.3).half().cuda()
    stages.append(C.stage(Xd, qw, bias=bias, strip_cols=64))
    want.append(ng.matmul_bias(Xd, ng.to_strip_major(qw, 64), bias))
    _, _, _, Xd, gate = synthetic(M, ke, 2048, 128, seed=81)
    _, _, _, _, up = synthetic(M, ke, 2048, 128, seed=82)
    gu = ng.interleave_swiglu(gate, up)
    for sw in (32, 64):
        stages.append(C.stage(Xd, gu, swiglu=True, strip_cols=sw))
        want.append(ng.matmul_swiglu(Xd, ng.to_strip_major(gu, sw)))
    got = _run(C.DecodeChain(stages, M=M))
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), (M, i)
    # group size 64
    stages, want = [], []
    for i, (K, N, g, sw) in enumerate(cases):
        if g != 64 or K > kmax:
            continue
        _, _, _, Xd, qw = synthetic(M, K, N, g, seed=90 + i)
        stages.append(C.stage(Xd, qw, strip_cols=sw))
        want.append(ng.matmul(Xd, ng.to_strip_major(qw, sw)))
    got = _run(C.DecodeChain(stages, M=M))
    assert all(torch.equal(a, b) for a, b in zip(got, want))


@pytest.mark.gpu
def test_packed_dependent_stages():
    """A dependent chain on packed weights (each stage reads the one before):
    the bits of the same chain on strip-major copies."""
    _, _, _, Xd, w1 = synthetic(1, 4096, 4096, 128, seed=91)
    _, _, _, _, w2 = synthetic(1, 4096, 14336, 128, seed=92)
    _, _, _, _, w3 = synthetic(1, 14336, 4096, 128, seed=93)
    outs = []
    for conv in (False, True):
        ws = [ng.to_strip_major(w, C.chain_strip_cols(w.K, w.N, 128)) if conv else w
              for w in (w1, w2, w3)]
        s0 = C.stage(Xd, ws[0])
        s1 = C.stage(s0.Y, ws[1], after=0)
        s2 = C.stage(s1.Y, ws[2], after=1)
        outs.append(_run(C.DecodeChain([s0, s1, s2])))
    assert all(torch.equal(a, b) for a, b in zip(*outs))


@pytest.mark.gpu
def test_group_size_64_chain():
    stages, want = [], []
    for i, (K, N) in enumerate([(2048, 1024), (4096, 2048), (1024, 4096)]):
        _, _, _, Xd, qw = synthetic(1, K, N, 64, seed=60 + i)
        sm = ng.to_strip_major(qw)
        stages.append(C.stage(Xd, sm))
        want.append(ng.matmul(Xd, sm))
    got = _run(C.DecodeChain(stages))
    assert all(torch.equal(a, b) for a, b in zip(got, want))


def _dataflow(layers: int = 2):
    built = D.build_layers(layers, seed=7)
    sm = D.strips([D.fuse(layer, swiglu=True) for layer in built])
    return D.DataflowStep(sm)


@pytest.mark.gpu
def test_dependent_data_flow_of_two_full_layers():
    """q|k|v -> o (+ residual) -> SwiGLU gate|up -> down (+ residual) -> the
    next layer, every stage waiting for the one before it: the chain's 8
    outputs have the bits of the 8 per-projection launches."""
    df = _dataflow(2)
    want = df.step_outputs()
    chain = df.as_chain()
    assert chain.workgroups == torch.cuda.get_device_properties(0).multi_processor_count
    got = _run(chain)
    assert len(got) == 8
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), i
    # The outputs are the data flow's: the last is a finite [1, 4096] row.
    assert got[-1].shape == (1, 4096) and torch.isfinite(got[-1].float()).all()


@pytest.mark.gpu
def test_dependent_chain_graph_replays_repeat_eager_bits():
    df = _dataflow(2)
    chain = df.as_chain()
    eager = _run(chain)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        chain.run()
    other = D.DataflowStep(df.layers, seed=11)  # other eager work between replays
    for _ in range(3):
        for y in chain.outputs():
            y.zero_()
        other.step_outputs()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(chain.outputs(), eager):
            assert torch.equal(a, b)
    chain.check()


@pytest.mark.gpu
def test_many_runs_repeat_their_bits():
    """300 back-to-back runs: the stage counters return to zero after every
    run (the last workgroup resets them), so every run waits correctly."""
    df = _dataflow(1)
    chain = df.as_chain()
    first = _run(chain)
    for _ in range(300):
        chain.run()
    chain.check()
    assert all(torch.equal(a, b) for a, b in zip(chain.outputs(), first))


@pytest.mark.gpu
def test_timestamps_follow_the_dependencies():
    df = _dataflow(2)
    chain = df.as_chain()
    _run(chain)
    t = chain.new_timestamps()
    chain.run(t)
    chain.check()
    ends = C.DecodeChain.stage_times_us(t)
    assert all(e > 0 for e in ends)
    # each stage ends after the one it waited for
    assert all(b >= a for a, b in zip(ends, ends[1:]))
    assert ends[-1] < 1e4


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [False, True])
def test_persistent_step_on_packed_weights(fused):
    """The reference-semantics step of two full layers (its 7 projections
    each, or the fused 4) as one chain straight on the packed (drop-in)
    weights: the bits of the chain on strip-major copies at the same widths."""
    layers = D.build_layers(2, seed=9)
    if fused:
        layers = [D.fuse(layer) for layer in layers]
    launches = D.DecodeStep(layers)
    packed = C.DecodeChain(D.chain_stages(layers, launches.acts))
    copies = D.strips(layers, chain=True)
    strip = C.DecodeChain(D.chain_stages(copies, launches.acts))
    got, want = _run(packed), _run(strip)
    assert len(got) == (8 if fused else 14)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    # replayed from a HIP graph, with the strip-major chain run between replays
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        packed.run()
    for _ in range(3):
        for y in packed.outputs():
            y.fill_(float("nan"))
        strip.run()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(packed.outputs(), want))
    packed.check()


@pytest.mark.gpu
@pytest.mark.parametrize("chain_widths,tp", [(False, 1), (True, 1), (True, 8)])
def test_persistent_step_matches_the_fused_launches(chain_widths, tp):
    """The reference-semantics step (independent projections) of two full
    layers -- or of one GPU's share of an 8-way split of them -- as one
    chain: the bits of the fused strip-major launches on the same copy, at
    the launches' strip widths or at the chain's."""
    built = D.build_layers(2, seed=8, tp=tp)
    fs = D.strips([D.fuse(layer) for layer in built], chain=chain_widths)
    widths = {name: w.strip_cols for name, w in fs[0].items()}
    assert widths == ({"qkv": 64, "o": 64, "gate_up": 64, "down": 32 if tp == 1 else 64}
                      if chain_widths else {"qkv": 32, "o": 16, "gate_up": 64, "down": 16})
    launches = D.DecodeStep(fs)
    chain = C.DecodeChain(D.chain_stages(fs, launches.acts))
    got = D.ChainStep(chain, D.weight_bytes(fs)).outputs()
    chain.check()
    want = launches.outputs()
    assert len(got) == len(want) == 8
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    # replayed from a HIP graph, with other eager work between the replays
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        chain.run()
    for _ in range(3):
        for y in chain.outputs():
            y.fill_(float("nan"))
        launches.outputs()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(chain.outputs(), want))
    chain.check()


@pytest.mark.gpu
def test_a_few_stages_leave_workgroups_idle():
    """One small stage: most workgroups have no round and finish at once."""
    X, packed, scales, Xd, qw = synthetic(1, 1024, 256, 128, seed=70)
    sm = ng.to_strip_major(qw, 32)
    chain = C.DecodeChain([C.stage(Xd, sm)])
    assert chain.rounds == 256 // 32
    got = _run(chain)[0]
    assert torch.equal(got, ng.matmul(Xd, sm))
    assert rms_err(host(got), oracle_y(X, packed, scales, 1024, 128)) <= 1e-2
