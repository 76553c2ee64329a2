"""Decode-step glue: RMSNorm and grouped-query attention kernels, and a whole
Llama-shaped token step built from them and the W4A16 projections.

The references are plain PyTorch in float32 (these are floating-point kernels
with no counterpart in the reference's extension; its model decode runs them
as transformers ops, bench/bench_model.py:177-188).  The CPU tests cover the
library's argument checks, which run before any HIP call.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import nibblegemm_amd as ng
from nibblegemm_amd import glue
from nibblegemm_amd.quant import split_swiglu

INVALID, WORKSPACE = 1, 3
P = 1 << 20  # aligned, never dereferenced
dev = "cuda"


# ---------------------------------------------------------------------------
# argument checks (CPU)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,eps,needle", [
    (1, 4100, 1e-5, "multiple of 8"),
    (1, 0, 1e-5, "multiple of 8"),
    (1, 16392, 1e-5, "up to 16384"),
    (-1, 4096, 1e-5, "rows"),
    (1, 4096, -1.0, "eps"),
    (1, 4096, float("nan"), "eps"),
])
def test_rmsnorm_rejections(rows, cols, eps, needle):
    ext = ng.extension()
    assert ext.rmsnorm(P, rows, cols, P, eps, P, None) == INVALID
    assert needle in ext.last_error()


def test_rmsnorm_rejects_misaligned_and_null():
    ext = ng.extension()
    assert ext.rmsnorm(P + 8, 1, 4096, P, 1e-5, P, None) == INVALID
    assert "aligned" in ext.last_error()
    assert ext.rmsnorm(0, 1, 4096, P, 1e-5, P, None) == INVALID
    assert "null" in ext.last_error()
    assert ext.rmsnorm(0, 0, 4096, 0, 1e-5, 0, None) == 0  # no rows: nothing to touch


def attn(ext, nh=32, nkv=8, hd=128, ms=2048, pos=1023, cos=None, sin=None, ws=None, wsb=0,
         ptr=P):
    return ext.attention(ptr, nh, nkv, hd, ptr, ptr, ms, pos, cos, sin, ptr, ws, wsb, None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(hd=64), "head_dim"),
    (dict(nh=30), "multiple of n_kv_heads"),
    (dict(nh=48, nkv=4), "1, 2, 4 or 8"),
    (dict(nkv=0), "n_kv_heads"),
    (dict(pos=2048), "pos"),
    (dict(pos=-1), "pos"),
    (dict(ms=(1 << 16) + 1, pos=5), "max_seq"),
    (dict(cos=P), "both"),
    (dict(pos=5, ptr=P + 2), "aligned"),
    (dict(pos=5, ptr=0), "null"),
])
def test_attention_rejections(kwargs, needle):
    ext = ng.extension()
    assert attn(ext, **kwargs) == INVALID
    assert needle in ext.last_error()


def test_attention_workspace_plan():
    """Up to 128 tokens run in one workgroup per kv head and need no
    workspace; beyond, chunks of 128 tokens publish (max, sum, 128 partial
    outputs) per query head, after a 256-byte counter block."""
    ext = ng.extension()
    assert ext.attention_workspace_bytes(32, 8, 128, 4096, 0, None) == (0, 0)
    assert ext.attention_workspace_bytes(32, 8, 128, 4096, 127, None) == (0, 0)
    assert ext.attention_workspace_bytes(32, 8, 128, 4096, 128, None) == \
        (256 + 8 * 2 * 4 * 130 * 4, 256)
    assert ext.attention_workspace_bytes(32, 8, 128, 4096, 1023, None) == \
        (256 + 8 * 8 * 4 * 130 * 4, 256)
    assert ext.attention_workspace_bytes(8, 8, 128, 4096, 300, None) == \
        (256 + 8 * 3 * 1 * 130 * 4, 256)
    assert ext.attention_workspace_bytes(32, 8, 64, 4096, 300, None) == (0, 0)  # rejected plan
    assert attn(ext, pos=1023, ws=None) == WORKSPACE
    assert "workspace" in ext.last_error()
    assert attn(ext, pos=1023, ws=P, wsb=1000) == WORKSPACE
    assert attn(ext, pos=1023, ws=P + 64, wsb=1 << 20) == WORKSPACE
    assert "256-byte" in ext.last_error()


def test_rope_tables_match_the_closed_form():
    cos, sin = glue.rope_tables(5, device="cpu")
    assert cos.shape == (5, 64) and cos.dtype == torch.float32
    for p in (0, 1, 4):
        for i in (0, 1, 17, 63):
            ang = p * 500000.0 ** (-2 * i / 128)
            assert cos[p, i].item() == pytest.approx(math.cos(ang), abs=1e-7)
            assert sin[p, i].item() == pytest.approx(math.sin(ang), abs=1e-7)


# ---------------------------------------------------------------------------
# references (float32)
# ---------------------------------------------------------------------------
def ref_rmsnorm(x, w, eps):
    xf = x.float()
    r = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * r * w.float()).half()


def ref_rope(x, cos, sin):
    """x float32 [H, 128]; cos, sin float32 [64] (transformers' rotate_half)."""
    x1, x2 = x[:, :64], x[:, 64:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=1)


def ref_attention(qkv, kc, vc, pos, n_heads, n_kv, rope=None):
    """Returns (out fp16 [1, n_heads * 128], k row fp16 [n_kv, 128], v row)."""
    q = qkv[0, :n_heads * 128].float().view(n_heads, 128)
    k = qkv[0, n_heads * 128:(n_heads + n_kv) * 128].float().view(n_kv, 128)
    v = qkv[0, (n_heads + n_kv) * 128:].view(n_kv, 128)
    if rope is not None:
        cos, sin = rope[0][pos].float(), rope[1][pos].float()
        q, k = ref_rope(q, cos, sin), ref_rope(k, cos, sin)
    knew = k.half()
    K = torch.cat([kc[:, :pos].float(), knew.float()[:, None]], dim=1)
    V = torch.cat([vc[:, :pos].float(), v.float()[:, None]], dim=1)
    qpk = n_heads // n_kv
    K = K.repeat_interleave(qpk, dim=0).contiguous()
    V = V.repeat_interleave(qpk, dim=0).contiguous()
    s = torch.bmm(K, q[:, :, None].contiguous())[:, :, 0] / math.sqrt(128)
    p = torch.softmax(s, dim=-1)
    out = torch.bmm(p[:, None, :].contiguous(), V)[:, 0]
    return out.reshape(1, -1).half(), knew, v


def err_rms(y, ref):
    ref = ref.float()
    return float((y.float() - ref).abs().max() / ref.pow(2).mean().sqrt())


def ulp_excess(y, ref, rel_rms=1e-3):
    """max of |y - ref| / (one fp16 ulp of ref + rel_rms * rms(ref)): <= 1
    when y differs from the fp32 reference by its own output rounding only
    (fp32 summation-order effects are far below the margin)."""
    ref = ref.float()
    tol = torch.finfo(torch.float16).eps * ref.abs() + rel_rms * ref.pow(2).mean().sqrt()
    return float(((y.float() - ref).abs() / tol).max())


# ---------------------------------------------------------------------------
# kernels (GPU)
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(1, 4096), (3, 4096), (2, 8), (1, 1000), (2, 16384),
                                       (5, 2056)])
def test_rmsnorm_matches_fp32(rows, cols):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn((rows, cols), generator=g) * 3).half().to(dev)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).half().to(dev)
    y = glue.rmsnorm(x, w, 1e-5)
    ref = ref_rmsnorm(x, w, 1e-5)
    # one rounding to fp16 after fp32 math: at most one fp16 ulp apart
    ulp = torch.finfo(torch.float16).eps * ref.float().abs().clamp_min(2.0 ** -14)
    assert bool(((y.float() - ref.float()).abs() <= ulp).all())
    assert (y == ref).float().mean().item() > 0.98


@pytest.mark.gpu
def test_rmsnorm_empty_and_zero_rows():
    w = torch.ones(64, dtype=torch.float16, device=dev)
    assert glue.rmsnorm(torch.empty((0, 64), dtype=torch.float16, device=dev), w).shape == (0, 64)
    z = glue.rmsnorm(torch.zeros((1, 64), dtype=torch.float16, device=dev), w, 1e-5)
    assert bool((z == 0).all())


def _attn_case(n_heads, n_kv, pos, max_seq, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn((1, (n_heads + 2 * n_kv) * 128), generator=g).half().to(dev)
    kc = torch.randn((n_kv, max_seq, 128), generator=g).half().to(dev)
    vc = torch.randn((n_kv, max_seq, 128), generator=g).half().to(dev)
    return qkv, kc, vc


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads,n_kv", [(32, 8), (8, 8), (16, 8), (64, 8)])
@pytest.mark.parametrize("pos", [0, 1, 127, 128, 129, 300, 1023])
@pytest.mark.parametrize("use_rope", [True, False])
def test_attention_matches_fp32(n_heads, n_kv, pos, use_rope):
    max_seq = 1040
    qkv, kc, vc = _attn_case(n_heads, n_kv, pos, max_seq, seed=pos * 31 + n_heads)
    rope = glue.rope_tables(max_seq) if use_rope else None
    ref, knew, vnew = ref_attention(qkv, kc, vc, pos, n_heads, n_kv, rope)
    before = (kc.clone(), vc.clone())
    out = glue.attention_decode(qkv, kc, vc, pos, rope)
    assert out.shape == (1, n_heads * 128)
    assert err_rms(out, ref) <= 1e-2
    assert ulp_excess(out, ref) <= 1.0, ulp_excess(out, ref)
    # row pos now holds the token's (rotated) k and its v; nothing else changed
    assert torch.equal(vc[:, pos], vnew)
    kd = (kc[:, pos].float() - knew.float()).abs()
    assert bool((kd <= torch.finfo(torch.float16).eps * knew.float().abs().clamp_min(2.0 ** -14)).all())
    mask = torch.ones(max_seq, dtype=torch.bool)
    mask[pos] = False
    assert torch.equal(kc[:, mask], before[0][:, mask]) and torch.equal(vc[:, mask], before[1][:, mask])


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads", [32, 64, 8])
def test_attention_long_context_and_repeat(n_heads):
    """4096 tokens (32 chunks per kv head, more than the combine loads in its
    first round for every head ratio); a second call gives the same bits
    (the combine order is fixed and the counters were restored)."""
    n_kv, pos, max_seq = 8, 4095, 4096
    qkv, kc, vc = _attn_case(n_heads, n_kv, pos, max_seq, seed=5)
    rope = glue.rope_tables(max_seq)
    ref, _, _ = ref_attention(qkv, kc, vc, pos, n_heads, n_kv, rope)
    a = glue.attention_decode(qkv, kc, vc, pos, rope)
    b = glue.attention_decode(qkv, kc, vc, pos, rope)
    assert err_rms(a, ref) <= 1e-2
    assert ulp_excess(a, ref) <= 1.0, ulp_excess(a, ref)
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_attention_combine_repeats_its_bits():
    """1024 tokens (8 chunks per kv head, combined by the last workgroup to
    arrive), 300 calls back to back: identical bits each time."""
    n_heads, n_kv, pos, max_seq = 32, 8, 1023, 1024
    qkv, kc, vc = _attn_case(n_heads, n_kv, pos, max_seq, seed=13)
    rope = glue.rope_tables(max_seq)
    first = glue.attention_decode(qkv, kc, vc, pos, rope)
    outs = [glue.attention_decode(qkv, kc, vc, pos, rope) for _ in range(300)]
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(y, first)


@pytest.mark.gpu
def test_attention_single_token_is_v():
    """At position 0 the softmax has one entry: the output is v itself
    (each query head reading its kv head)."""
    qkv, kc, vc = _attn_case(32, 8, 0, 16, seed=9)
    out = glue.attention_decode(qkv, kc, vc, 0, glue.rope_tables(16))
    v = qkv[0, 40 * 128:].view(8, 128)
    assert torch.equal(out.view(32, 128), v.repeat_interleave(4, dim=0))


@pytest.mark.gpu
def test_attention_graph_replay():
    n_heads, n_kv, pos, max_seq = 32, 8, 700, 1024
    qkv, kc, vc = _attn_case(n_heads, n_kv, pos, max_seq, seed=3)
    rope = glue.rope_tables(max_seq)
    eager = glue.attention_decode(qkv, kc, vc, pos, rope)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        glue.attention_decode(qkv, kc, vc, pos, rope)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = glue.attention_decode(qkv, kc, vc, pos, rope)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        glue.attention_decode(qkv, kc, vc, pos, rope)  # eager work between replays


# ---------------------------------------------------------------------------
# a whole token step
# ---------------------------------------------------------------------------
def ref_step(step, layers):
    """The step in float32 with fp16 storage at every op boundary (the
    roundings of the fp16 model's separate ops)."""
    hs = step.x
    for layer, (wa, wf), (kc, vc) in zip(layers, step.norms, step.caches):
        W = {k: ng.dequant(qw).float() for k, qw in layer.items()}  # bit-exact, tested
        a = ref_rmsnorm(hs, wa, step.eps)
        qkv = (a.float() @ W["qkv"]).half()
        att, _, _ = ref_attention(qkv, kc, vc, step.pos, 32, 8, step.rope)
        h1 = (hs.float() + (att.float() @ W["o"]).half().float()).half()
        b = ref_rmsnorm(h1, wf, step.eps)
        gate, up = split_swiglu((b.float() @ W["gate_up_swiglu"]).half())
        m = F.silu(gate) * up
        hs = (h1.float() + (m.float() @ W["down"]).half().float()).half()
    return hs


@pytest.mark.gpu
@pytest.mark.parametrize("n_layers,pos", [(1, 0), (1, 300), (2, 129)])
def test_glue_step_matches_fp32(n_layers, pos):
    from nibblegemm_amd import decode_step as D
    layers = [D.fuse(layer, swiglu=True) for layer in D.build_layers(n_layers, seed=11)]
    step = D.GlueDecodeStep(layers, pos=pos, max_seq=pos + 8)
    y = step()  # writes cache row pos only; the reference reads rows < pos
    assert step.launches == 5 * n_layers
    ref = ref_step(step, layers)
    assert err_rms(y, ref) <= 1e-2, err_rms(y, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(1, 4096, 6144), (1, 4096, 4096), (2, 16384, 512),
                                   (3, 1024, 1024), (8, 4096, 2048), (1, 128, 64)])
@pytest.mark.parametrize("epi", ["none", "bias", "swiglu"])
def test_rmsnorm_matmul_fused_is_the_two_step_bits(M, K, N, epi):
    """The streaming kernel's RMSNorm prologue reproduces the RMSNorm
    kernel's row scale and rounding, so the fused launch gives exactly the
    bits of rmsnorm followed by the matmul (and its epilogue)."""
    from nibblegemm_amd import ops
    g = torch.Generator().manual_seed(M * 131 + K + N)
    qw = ng.quantize((torch.randn((K, N), generator=g) * 0.02), 128).to(dev)
    x = (torch.randn((M, K), generator=g) * 2).half().to(dev)
    w = (1 + 0.1 * torch.randn(K, generator=g)).half().to(dev)
    bias = torch.randn(N, generator=g).half().to(dev) if epi == "bias" else None
    fused = ops.rmsnorm_matmul(x, w, qw, 1e-5, bias=bias, swiglu=epi == "swiglu")
    # the one-launch form directly, also where rmsnorm_matmul composes (M > 3)
    code = 2 if epi == "swiglu" else 1 if epi == "bias" else 0
    direct = ops._fused(x, qw, code, bias, N // 2 if epi == "swiglu" else N, (w, 1e-5))
    a = glue.rmsnorm(x, w, 1e-5)
    if epi == "swiglu":
        ref = ops.matmul_swiglu(a, qw)
    elif epi == "bias":
        ref = ops.matmul_bias(a, qw, bias)
    else:
        ref = ops.matmul(a, qw)
    assert torch.equal(fused, ref)
    assert torch.equal(direct, ref)
    W = ng.dequant(qw).float()
    if epi == "none":
        assert err_rms(fused, (a.float() @ W).half()) <= 1e-2


@pytest.mark.gpu
def test_rmsnorm_matmul_beyond_the_fused_limits_composes():
    from nibblegemm_amd import ops
    g = torch.Generator().manual_seed(4)
    qw = ng.quantize(torch.randn((1024, 256), generator=g) * 0.02, 128).to(dev)
    x = torch.randn((12, 1024), generator=g).half().to(dev)  # M > 3: two launches
    w = (1 + 0.1 * torch.randn(1024, generator=g)).half().to(dev)
    assert torch.equal(ops.rmsnorm_matmul(x, w, qw), ops.matmul(glue.rmsnorm(x, w), qw))


@pytest.mark.gpu
def test_glue_step_fused_norms_are_the_separate_launches():
    from nibblegemm_amd import decode_step as D
    layers = [D.fuse(layer, swiglu=True) for layer in D.build_layers(2, seed=13)]
    fused = D.GlueDecodeStep(layers, pos=150, fuse_norm=True)
    plain = D.GlueDecodeStep(layers, pos=150, fuse_norm=False)
    assert fused.launches == 10 and plain.launches == 14
    assert torch.equal(fused(), plain())


@pytest.mark.gpu
def test_glue_step_graph_replay():
    from nibblegemm_amd import decode_step as D
    layers = [D.fuse(layer, swiglu=True) for layer in D.build_layers(2, seed=12)]
    step = D.GlueDecodeStep(layers, pos=200)
    eager = step()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        step()
