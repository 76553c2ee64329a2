"""Llama-3-8B-shaped batch-1 decode step: every W4A16 projection of 32
layers, replayed from a HIP graph (the decode-step benchmark; the reference's
``bench/bench_model.py`` layers mode, :43-125).

Like the reference, a step is the projections only: q, k, v, o, gate, up and
down of every layer (224 ``matmul`` calls at M = 1), each reading activations
allocated once outside the timed region (bench_model.py:70-86).  Unlike the
reference, the 32 layers hold 32 *distinct* weight sets.  One INT4 layer is
~112 MB, which the reference could replay on an A100 because it exceeds that
part's 40 MB L2 (bench_model.py:50-56); on MI355X it would be served from the
256 MiB Infinity Cache, so replaying one layer would not measure HBM
streaming.

Weights are random-init ``randn * 0.02`` (bench_model.py:62), RTN-quantised
on the GPU by :func:`~nibblegemm_amd.quant.quantize_device` (bit-identical to
the host quantiser).

The fused variant concatenates q|k|v and gate|up along N
(:func:`~nibblegemm_amd.quant.concat_columns`), so a layer is 4 launches
instead of 7: 128 per step instead of 224.  ``fused_swiglu`` interleaves
gate and up instead and runs them through the SwiGLU epilogue
(:func:`~nibblegemm_amd.ops.matmul_swiglu`), whose launch writes the
[1, 14336] input of down directly.  The arithmetic is identical
(each output column is computed from the same weights, scales and
activations); it only removes launches.

The ``*_strips`` variants run the same steps on strip-major copies of the
weights (:func:`~nibblegemm_amd.ops.to_strip_major`, the decode GEMV's
contiguous-strip layout; same codes and scales, so the same bytes per
step).

``glue`` runs a whole token step instead (:class:`GlueDecodeStep`): per
layer RMSNorm, the q|k|v projection, rotary embedding and grouped-query
attention over a KV cache of ``pos`` tokens, the o projection with the
residual add in its epilogue, RMSNorm, gate|up through the SwiGLU epilogue
and the down projection with the second residual add, every one a kernel of
this library.  Each RMSNorm runs as the prologue of the projection after it
(:func:`~nibblegemm_amd.ops.rmsnorm_matmul`, the same bits as the separate
launch), so a layer is 5 launches.  This is the per-token forward of
the reference's model decode (bench/bench_model.py:177-188) without the
embedding lookup and the fp16 lm_head, which are not W4A16.

``persistent_projections`` runs the reference's step itself -- the 224
separate projections on strip-major weights, each reading its fixed
activation -- as ONE launch; ``persistent`` runs the fused strip-major step
the same way: a
:class:`~nibblegemm_amd.chain.DecodeChain` of the 128 projections, each still
reading its fixed activation (the reference's semantics), whose workgroups
stream weights across projection boundaries.  Both run on strip-major copies
at the chain's widths (:func:`~nibblegemm_amd.chain.chain_strip_cols`: 64
columns, down 32, where the launches take 16 to 64), and their outputs are
bit-identical to the launches on the same copy.  ``persistent_packed`` and
``persistent_projections_packed`` run the same chains straight on the packed
weights, the drop-in layout, unconverted (the bits of the chains on
strip-major copies).  ``dataflow`` is the real data flow of a decoder layer
without attention and norms, one launch per projection on strip-major
weights: the q|k|v product, o on its q part with the layer input added as
the residual, gate|up through the SwiGLU epilogue, and down with o's output
added, whose result is the next layer's input.  ``persistent_dataflow`` runs
that same dependent sequence as one chain (every stage waits for the one
before it) with the same bits.

``--tp N`` builds every layer at one GPU's share of an N-way tensor-parallel
split instead (:func:`projection_shapes`): q, k, v, gate and up split by
columns (N / tp each), o and down by rows (K / tp, whole quant groups).  It
times what one GPU's kernels cost per token at that split; the exchange a
row-split layer needs after o and down (an all-reduce of its partial
outputs) is not built, and the row-split projections here store fp16 where
a sharded layer would keep fp32 partials for that sum.  The glue variants
need every head and are full-model only.

    python -m nibblegemm_amd.decode_step --layers 32
    python -m nibblegemm_amd.decode_step --layers 32 --tp 8 --variants projections_strips,fused_strips
"""
from __future__ import annotations

import argparse
import json
import sys
from typing import Dict, List, Tuple

import torch

from . import harness as H
from .chain import DecodeChain, chain_strip_cols, stage
from .glue import attention_bytes, attention_decode, rmsnorm, rope_tables
from .ops import (matmul, matmul_bias, matmul_swiglu, rmsnorm_matmul, strip_major_cols,
                  to_strip_major)
from .quant import QuantizedWeight, concat_columns, interleave_swiglu, quantize_device

LLAMA3_8B = {"hidden": 4096, "kv": 1024, "intermediate": 14336, "layers": 32,
             "heads": 32, "kv_heads": 8, "rms_eps": 1e-5}
PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


#: Projections split by output columns under tensor parallelism (the rest,
#: o and down, split by input rows).
COLUMN_SPLIT = ("q", "k", "v", "gate", "up")


def projection_shapes(cfg=LLAMA3_8B, tp: int = 1,
                      group_size: int = 128) -> Dict[str, Tuple[int, int]]:
    """(K, N) of every projection, consumed as ``Y = X @ W`` (bench_model.py:57-59),
    at one GPU's share of a ``tp``-way tensor-parallel split: N / tp for the
    column-split projections, K / tp for o and down.  Column shares must stay
    multiples of 16 (whole SwiGLU blocks) and row shares whole quant groups."""
    h, kv, inter = cfg["hidden"], cfg["kv"], cfg["intermediate"]
    full = {"q": (h, h), "k": (h, kv), "v": (h, kv), "o": (h, h),
            "gate": (h, inter), "up": (h, inter), "down": (inter, h)}
    if tp < 1:
        raise ValueError(f"tp={tp} must be >= 1")
    out = {}
    for name, (K, N) in full.items():
        if name in COLUMN_SPLIT:
            if N % (16 * tp):
                raise ValueError(f"{name}: N={N} does not split {tp} ways in 16-column blocks")
            out[name] = (K, N // tp)
        else:
            if K % (group_size * tp):
                raise ValueError(f"{name}: K={K} does not split {tp} ways in groups of {group_size}")
            out[name] = (K // tp, N)
    return out


def build_layers(layers: int, cfg=LLAMA3_8B, group_size: int = 128, device="cuda",
                 seed: int = 0, tp: int = 1) -> List[Dict[str, QuantizedWeight]]:
    """``layers`` distinct sets of RTN-quantised projections, built on the GPU
    (at one GPU's ``tp``-way share, :func:`projection_shapes`)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    shapes = projection_shapes(cfg, tp, group_size)
    out = []
    for _ in range(layers):
        layer = {}
        for name in PROJECTIONS:
            K, N = shapes[name]
            W = torch.randn((K, N), generator=gen, device=device, dtype=torch.float32) * 0.02
            layer[name] = quantize_device(W, group_size)
            del W
        out.append(layer)
    return out


def fuse(layer: Dict[str, QuantizedWeight], swiglu: bool = False) -> Dict[str, QuantizedWeight]:
    """q|k|v and gate|up concatenated along N; o and down unchanged.  With
    ``swiglu`` gate and up are interleaved for the SwiGLU epilogue instead
    (the launch then writes silu(gate) * up, [1, 14336], for down)."""
    gate_up = (interleave_swiglu(layer["gate"], layer["up"]) if swiglu
               else concat_columns(layer["gate"], layer["up"]))
    return {"qkv": concat_columns(layer["q"], layer["k"], layer["v"]), "o": layer["o"],
            ("gate_up_swiglu" if swiglu else "gate_up"): gate_up, "down": layer["down"]}


def strips(layers: List[Dict[str, QuantizedWeight]], chain: bool = False) -> list:
    """Strip-major copies of every weight, each at the width the launches
    stream fastest (``strip_major_cols``) or, with ``chain``, the width a
    decode chain does (``chain_strip_cols``: 64 or 32 columns where they fit;
    MI355X, 8B step as one chain, 0.585 -> 0.552 ms with o and down at 32
    columns instead of 16, while the 128 launches go 0.892 -> 0.955 ms).
    The SwiGLU weight takes at least 32 columns either way: its strips must
    hold whole gate|up block pairs."""
    def one(name, qw):
        sw = (chain_strip_cols if chain else strip_major_cols)(qw.K, qw.N, qw.group_size)
        return to_strip_major(qw, max(sw, 32) if name == "gate_up_swiglu" else sw)
    return [{name: one(name, qw) for name, qw in layer.items()} for layer in layers]


def weight_bytes(layers: List[Dict[str, QuantizedWeight]]) -> int:
    return sum(qw.weight_bytes for layer in layers for qw in layer.values())


class DecodeStep:
    """One step's matmul calls, with activations allocated once."""

    def __init__(self, layers: List[Dict[str, QuantizedWeight]], device="cuda", seed: int = 1):
        gen = torch.Generator(device=device).manual_seed(seed)
        ks = sorted({qw.K for layer in layers for qw in layer.values()})
        self.acts = {k: torch.randn((1, k), generator=gen, device=device).to(torch.float16)
                     for k in ks}
        self.calls = [(self.acts[qw.K], qw, matmul_swiglu if name == "gate_up_swiglu" else matmul)
                      for layer in layers for name, qw in layer.items()]

    def __call__(self, _i: int = 0) -> None:
        for x, qw, fn in self.calls:
            fn(x, qw)

    def outputs(self) -> List[torch.Tensor]:
        """The step with every call's output kept, in call order."""
        return [fn(x, qw) for x, qw, fn in self.calls]

    @property
    def launches(self) -> int:
        return len(self.calls)


def chain_stages(layers: List[Dict[str, QuantizedWeight]], acts: Dict[int, torch.Tensor]) -> list:
    """The projections of ``layers`` (strip-major weights, or packed ones read
    as strips of the chain's widths) as independent chain stages, each
    reading its fixed activation ``acts[K]`` (the reference's decode-step
    semantics) and writing its own output."""
    out = []
    for layer in layers:
        for name, w in layer.items():
            out.append(stage(acts[w.K], w, swiglu=name == "gate_up_swiglu"))
    return out


class ChainStep:
    """A decode step run as one :class:`DecodeChain` launch."""

    def __init__(self, chain: DecodeChain, nbytes: int):
        self.chain = chain
        self.nbytes = nbytes

    def __call__(self, _i: int = 0) -> None:
        self.chain.run()

    def outputs(self) -> List[torch.Tensor]:
        self.chain.run()
        return [y.clone() for y in self.chain.outputs()]

    @property
    def launches(self) -> int:
        return 1


class DataflowStep:
    """The data flow of a decoder layer without attention and norms, one
    launch per projection: ``qkv = x W_qkv``; ``h = q W_o + x`` (q the first
    ``hidden`` columns of qkv; the residual add as the fused bias);
    ``g = silu(h W_gate) * (h W_up)``; ``x' = g W_down + h``.  ``layers`` are
    ``fuse(layer, swiglu=True)`` sets (strip-major or packed).  A call makes
    the launches alone (outputs from the caching allocator, as any
    ``matmul``); :meth:`as_chain` builds the same step as one chain writing
    into buffers allocated once here."""

    def __init__(self, layers: List[Dict[str, QuantizedWeight]], cfg=LLAMA3_8B, device="cuda",
                 seed: int = 3):
        gen = torch.Generator(device=device).manual_seed(seed)
        h, inter = cfg["hidden"], cfg["intermediate"]
        self.layers = layers
        self.hidden = h
        self.x0 = torch.randn((1, h), generator=gen, device=device).to(torch.float16)
        self.bufs = []
        for layer in layers:
            nqkv = layer["qkv"].N
            self.bufs.append({"qkv": torch.empty((1, nqkv), dtype=torch.float16, device=device),
                              "h": torch.empty((1, h), dtype=torch.float16, device=device),
                              "g": torch.empty((1, inter), dtype=torch.float16, device=device),
                              "x": torch.empty((1, h), dtype=torch.float16, device=device)})

    def __call__(self, _i: int = 0) -> None:
        self.step_outputs()

    def step_outputs(self) -> List[torch.Tensor]:
        """One step's four activations of every layer, in order."""
        out, x = [], self.x0
        for layer in self.layers:
            qkv = matmul(x, layer["qkv"])
            hh = matmul_bias(qkv[:, :self.hidden], layer["o"], x.view(-1))
            g = matmul_swiglu(hh, layer["gate_up_swiglu"])
            x = matmul_bias(g, layer["down"], hh.view(-1))
            out += [qkv, hh, g, x]
        return out

    outputs = step_outputs

    def as_chain(self) -> DecodeChain:
        """The same step as one chain writing the same buffers: every stage
        waits for the one before it."""
        stages, x, prev = [], self.x0, -1
        for layer, b in zip(self.layers, self.bufs):
            stages.append(stage(x, layer["qkv"], after=prev, Y=b["qkv"]))
            stages.append(stage(b["qkv"][:, :self.hidden], layer["o"], bias=x.view(-1),
                                after=len(stages) - 1, Y=b["h"]))
            stages.append(stage(b["h"], layer["gate_up_swiglu"], swiglu=True,
                                after=len(stages) - 1, Y=b["g"]))
            stages.append(stage(b["g"], layer["down"], bias=b["h"].view(-1),
                                after=len(stages) - 1, Y=b["x"]))
            x, prev = b["x"], len(stages) - 1
        return DecodeChain(stages)

    def buffers(self) -> List[torch.Tensor]:
        return [b[k] for b in self.bufs for k in ("qkv", "h", "g", "x")]

    @property
    def launches(self) -> int:
        return 4 * len(self.layers)


class GlueDecodeStep:
    """One batch-1 token step of a Llama-shaped decoder at position ``pos``.

    ``layers`` are ``fuse(layer, swiglu=True)`` weight sets.  Each layer owns
    RMSNorm weights (``1 + 0.05 randn``), and k / v caches
    [kv_heads, max_seq, 128] whose rows ``0 .. pos - 1`` hold ``randn``
    (earlier tokens); a step writes row ``pos`` of each.  Replaying a step
    recomputes the same token at the same position.  The residual stream
    enters as ``x`` (a ``randn`` row, the embedding lookup's stand-in).  At
    M = 1 each residual add is the bias of the o / down projection's fused
    epilogue: ``fp16(fp16(a @ W) + h)``, the bits of the separate adds.
    """

    def __init__(self, layers: List[Dict[str, QuantizedWeight]], pos: int = 1023,
                 max_seq: int = 0, cfg=LLAMA3_8B, rope: bool = True, fuse_norm: bool = True,
                 device="cuda", seed: int = 2):
        gen = torch.Generator(device=device).manual_seed(seed)
        h, kvh = cfg["hidden"], cfg["kv_heads"]
        self.pos = int(pos)
        self.max_seq = int(max_seq) or self.pos + 1
        self.eps = float(cfg["rms_eps"])
        self.layers = layers
        self.x = torch.randn((1, h), generator=gen, device=device).to(torch.float16)
        self.norms = []
        self.caches = []
        for _ in layers:
            self.norms.append(tuple(
                (1.0 + 0.05 * torch.randn(h, generator=gen, device=device)).to(torch.float16)
                for _ in range(2)))
            kc = torch.zeros((kvh, self.max_seq, 128), dtype=torch.float16, device=device)
            vc = torch.zeros_like(kc)
            kc[:, :self.pos] = torch.randn((kvh, self.pos, 128), generator=gen, device=device)
            vc[:, :self.pos] = torch.randn((kvh, self.pos, 128), generator=gen, device=device)
            self.caches.append((kc, vc))
        self.rope = rope_tables(self.max_seq, device=device) if rope else None
        self.kv_heads = kvh
        self.fuse_norm = fuse_norm

    def __call__(self, _i: int = 0) -> torch.Tensor:
        hs = self.x
        for layer, (w_attn, w_ffn), (kc, vc) in zip(self.layers, self.norms, self.caches):
            if self.fuse_norm:
                qkv = rmsnorm_matmul(hs, w_attn, layer["qkv"], self.eps)
            else:
                qkv = matmul(rmsnorm(hs, w_attn, self.eps), layer["qkv"])
            att = attention_decode(qkv, kc, vc, self.pos, self.rope)
            h1 = matmul_bias(att, layer["o"], hs.view(-1))
            if self.fuse_norm:
                g = rmsnorm_matmul(h1, w_ffn, layer["gate_up_swiglu"], self.eps, swiglu=True)
            else:
                g = matmul_swiglu(rmsnorm(h1, w_ffn, self.eps), layer["gate_up_swiglu"])
            hs = matmul_bias(g, layer["down"], h1.view(-1))
        return hs

    @property
    def launches(self) -> int:
        return (5 if self.fuse_norm else 7) * len(self.layers)

    def step_bytes(self) -> int:
        """Weights, caches and norm weights one step reads (activations aside)."""
        per_layer = attention_bytes(self.kv_heads, self.pos) + 2 * 2 * self.x.numel()
        return weight_bytes(self.layers) + len(self.layers) * per_layer


def outputs_of(step) -> List[torch.Tensor]:
    """The tensors one call of ``step`` produces, in order."""
    if hasattr(step, "outputs"):
        return step.outputs()
    return [step()]


def graph_matches_eager(step) -> bool:
    """Captures one call of ``step`` into a HIP graph, replays it, and
    compares every output with an eager call's, bit for bit."""
    eager = [t.clone() for t in outputs_of(step)]
    torch.cuda.synchronize()
    kept: List[torch.Tensor] = []

    def body(_i):
        kept[:] = outputs_of(step)

    runner = H.GraphRunner(body, reps=1, warmup=1)
    runner.graph.replay()
    torch.cuda.synchronize()
    same = _same(kept, eager)
    del runner, kept
    return same


def measure_step(step, nbytes: int, trials: int = 10, warmup: int = 3, **extra) -> dict:
    """Eager and graph-replayed time of one step, as the reference reports it
    (bench_model.py:100-113), after checking that a graph replay gives the
    eager call's outputs bit for bit (raises otherwise)."""
    if not graph_matches_eager(step):
        raise RuntimeError(f"{type(step).__name__}: graph replay differs from the eager step")
    eager = H.bench(step, reps=1, trials=trials, warmup=warmup)
    graph = H.bench_graph(step, reps=1, trials=trials, warmup=warmup)
    return {
        "launches": step.launches,
        **extra,
        "weights_gib": round(nbytes / 2**30, 3),
        "eager_ms": round(eager.median_ms, 4),
        "graph_ms": round(graph.median_ms, 4),
        "tok_s": round(1000.0 / eager.median_ms, 1),
        "graph_tok_s": round(1000.0 / graph.median_ms, 1),
        "graph_gbps": round(nbytes / (graph.median_ms * 1e-3) / 1e9, 1),
        "graph_equals_eager": True,
        "clock_mhz": graph.clocks.get("clock_mean_mhz"),
        "throttled": graph.clocks.get("throttled"),
    }


def measure_glue(layers: List[Dict[str, QuantizedWeight]], pos: int = 1023, trials: int = 10,
                 warmup: int = 3) -> dict:
    step = GlueDecodeStep(layers, pos=pos)
    r = measure_step(step, step.step_bytes(), trials, warmup, context=pos + 1)
    r["step_gib"] = r.pop("weights_gib")
    return r


def measure(layers: List[Dict[str, QuantizedWeight]], trials: int = 10, warmup: int = 3) -> dict:
    return measure_step(DecodeStep(layers), weight_bytes(layers), trials, warmup)


def _same(a: List[torch.Tensor], b: List[torch.Tensor]) -> bool:
    """Bit-for-bit equality of two lists of fp16 tensors (NaNs included)."""
    return len(a) == len(b) and all(
        x.shape == y.shape and torch.equal(x.view(torch.int16), y.view(torch.int16))
        for x, y in zip(a, b))


def stage_times(chain: DecodeChain, names: List[str], runs: int = 5) -> dict:
    """Where a chain's time goes, from the kernel's own timestamps: per
    projection name (the layer's stages in order), the median over ``runs``
    of the mean over layers of the time from the end of the stage before it
    to its own end, in us (its effective time in the step), and the step's
    total.  Eager runs after ~50 ms of untimed ones (:func:`harness.keep_busy`),
    so they start at the loaded clock."""
    H.keep_busy(chain.run, 0.05)
    chain.check()
    per = {n: [] for n in names}
    totals = []
    for _ in range(runs):
        t = chain.new_timestamps()
        chain.run(t)
        chain.check()
        ends = DecodeChain.stage_times_us(t)
        deltas = [ends[0]] + [b - a for a, b in zip(ends, ends[1:])]
        for j, n in enumerate(names):
            d = deltas[j::len(names)]
            per[n].append(sum(d) / len(d))
        totals.append(max(ends))
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    return {**{n: round(med(v), 2) for n, v in per.items()}, "total_us": round(med(totals), 1)}


def measure_persistent(layers_sm: List[Dict[str, QuantizedWeight]], trials: int = 10,
                       warmup: int = 3, with_stages: bool = False) -> dict:
    """The step of ``layers_sm`` (strip-major) as one chain launch with the
    reference's semantics, after checking its outputs against the
    per-projection launches bit for bit (raises otherwise)."""
    launches = DecodeStep(layers_sm)
    chain = DecodeChain(chain_stages(layers_sm, launches.acts))
    step = ChainStep(chain, weight_bytes(layers_sm))
    if not _same(step.outputs(), launches.outputs()):
        raise RuntimeError("persistent chain differs from the per-projection launches")
    chain.check()
    r = measure_step(step, step.nbytes, trials, warmup, stages=len(chain.stages),
                     workgroups=chain.workgroups, rounds=chain.rounds,
                     equals_per_projection_launches=True)
    if with_stages:
        r["stage_us"] = stage_times(chain, list(layers_sm[0]))
    chain.check()
    return r


def measure_persistent_packed(layers: List[Dict[str, QuantizedWeight]], trials: int = 10,
                              warmup: int = 3) -> dict:
    """The step of ``layers`` as one chain reading the packed weights (the
    reference's layout) unconverted, after checking its outputs bit for bit
    against the same chain on strip-major copies at the same widths (raises
    otherwise); the copies are freed before the timing."""
    launches = DecodeStep(layers)
    chain = DecodeChain(chain_stages(layers, launches.acts))
    step = ChainStep(chain, weight_bytes(layers))
    copies = strips(layers, chain=True)
    ref = DecodeChain(chain_stages(copies, launches.acts))
    same = _same(step.outputs(), ChainStep(ref, 0).outputs())
    ref.check()
    ref.close()
    del ref, copies
    if not same:
        raise RuntimeError("persistent chain on packed weights differs from the strip-major chain")
    chain.check()
    r = measure_step(step, step.nbytes, trials, warmup, stages=len(chain.stages),
                     workgroups=chain.workgroups, rounds=chain.rounds,
                     equals_strip_major_chain=True)
    chain.check()
    return r


def measure_dataflow(layers_sm: List[Dict[str, QuantizedWeight]], trials: int = 10,
                     warmup: int = 3, persistent: bool = True,
                     with_stages: bool = False) -> Dict[str, dict]:
    """The layer data flow (:class:`DataflowStep`) one launch per projection,
    and (``persistent``) as one chain, after checking the chain's outputs
    against the launches' bit for bit (raises otherwise)."""
    df = DataflowStep(layers_sm)
    nbytes = weight_bytes(layers_sm)
    out = {"dataflow_strips": measure_step(df, nbytes, trials, warmup)}
    if persistent:
        chain = df.as_chain()
        step = ChainStep(chain, nbytes)
        if not _same(step.outputs(), df.step_outputs()):
            raise RuntimeError("persistent data-flow chain differs from the per-projection launches")
        chain.check()
        out["persistent_dataflow"] = measure_step(
            step, nbytes, trials, warmup, stages=len(chain.stages), workgroups=chain.workgroups,
            rounds=chain.rounds, equals_per_projection_launches=True)
        if with_stages:
            out["persistent_dataflow"]["stage_us"] = stage_times(chain, list(layers_sm[0]))
        chain.check()
    return out


VARIANTS = ("projections", "fused", "fused_swiglu", "glue", "projections_strips", "fused_strips",
            "fused_swiglu_strips", "glue_strips", "persistent_projections",
            "persistent_projections_packed", "persistent", "persistent_packed", "dataflow_strips",
            "persistent_dataflow")


def run(n_layers: int = 32, group_size: int = 128, trials: int = 10, glue_pos: int = 1023,
        variants=VARIANTS, tp: int = 1, with_stages: bool = False) -> dict:
    want = set(variants)
    if tp > 1 and want & {"glue", "glue_strips", "dataflow_strips", "persistent_dataflow"}:
        raise ValueError("the glue and data-flow variants run the full model only (tp = 1)")
    layers = build_layers(n_layers, group_size=group_size, tp=tp)
    nbytes = weight_bytes(layers)
    share = "" if tp == 1 else f", one GPU's share of a {tp}-way tensor-parallel split"
    res = {"config": f"Llama-3-8B shapes{share}, {n_layers} distinct layers, g={group_size}, M=1",
           "tp": tp, "shapes": {k: list(v) for k, v in projection_shapes(tp=tp,
                                                                      group_size=group_size).items()},
           "roofline_tok_s": round(H.HBM_PEAK_GBPS * 1e9 / nbytes, 1)}
    if "projections" in want:
        res["projections"] = measure(layers, trials)
    # Launch variants run on copies at the launches' widths, chain variants on
    # copies at the chain's: a model converts its one copy for the path it runs.
    if "projections_strips" in want:
        ps = strips(layers)
        res["projections_strips"] = measure(ps, trials)
        del ps
    if "persistent_projections" in want:
        ps = strips(layers, chain=True)
        res["persistent_projections"] = measure_persistent(ps, trials, with_stages=with_stages)
        del ps
    if "persistent_projections_packed" in want:
        res["persistent_projections_packed"] = measure_persistent_packed(layers, trials)
    if want & {"fused", "fused_strips", "persistent", "persistent_packed"}:
        fused = [fuse(layer) for layer in layers]
        if "fused" in want:
            res["fused"] = measure(fused, trials)
        if "fused_strips" in want:
            fs = strips(fused)
            res["fused_strips"] = measure(fs, trials)
            del fs
        if "persistent" in want:
            fs = strips(fused, chain=True)
            res["persistent"] = measure_persistent(fs, trials, with_stages=with_stages)
            del fs
        if "persistent_packed" in want:
            res["persistent_packed"] = measure_persistent_packed(fused, trials)
        del fused
    swiglu_want = {"fused_swiglu", "glue", "fused_swiglu_strips", "glue_strips",
                   "dataflow_strips", "persistent_dataflow"}
    if want & swiglu_want:
        swiglu = [fuse(layer, swiglu=True) for layer in layers]
        del layers
        if "fused_swiglu" in want:
            res["fused_swiglu"] = measure(swiglu, trials)
        if "glue" in want and glue_pos >= 0:
            res["glue"] = measure_glue(swiglu, glue_pos, trials)
        if want & (swiglu_want - {"fused_swiglu", "glue"}):
            # The dependent data-flow chain stays on the launches' widths: each
            # of its stages waits for the one before, so a stage's strip count
            # sets how many CUs share it (32-column o and down: 1.628 -> 1.647 ms).
            swiglu_strips = strips(swiglu)
            del swiglu
            if "fused_swiglu_strips" in want:
                res["fused_swiglu_strips"] = measure(swiglu_strips, trials)
            if "glue_strips" in want and glue_pos >= 0:
                res["glue_strips"] = measure_glue(swiglu_strips, glue_pos, trials)
            if want & {"dataflow_strips", "persistent_dataflow"}:
                res.update(measure_dataflow(swiglu_strips, trials,
                                            persistent="persistent_dataflow" in want,
                                            with_stages=with_stages))
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--group-size", type=int, default=128)
    ap.add_argument("--trials", type=int, default=10)
    ap.add_argument("--glue-pos", type=int, default=1023,
                    help="position of the full-step (glue) variant's token; -1 skips it")
    ap.add_argument("--variants", default=None,
                    help="comma-separated subset of " + ", ".join(VARIANTS)
                    + " (default: all; with --tp > 1 all but the glue variants)")
    ap.add_argument("--tp", type=int, default=1,
                    help="time one GPU's share of a TP-way tensor-parallel split")
    ap.add_argument("--stage-times", action="store_true",
                    help="add each persistent chain's per-projection effective times "
                         "(in-kernel timestamps)")
    args = ap.parse_args(argv)
    default = VARIANTS if args.tp == 1 else tuple(
        v for v in VARIANTS if "glue" not in v and "dataflow" not in v)
    variants = tuple(v for v in args.variants.split(",") if v) if args.variants else default
    if not set(variants) <= set(VARIANTS):
        ap.error(f"unknown variant in {args.variants!r}")
    try:
        projection_shapes(tp=args.tp, group_size=args.group_size)
    except ValueError as e:
        ap.error(str(e))
    if args.tp > 1 and {"glue", "glue_strips", "dataflow_strips", "persistent_dataflow"} & set(variants):
        ap.error("the glue and data-flow variants run the full model only (tp = 1)")
    if not torch.cuda.is_available():
        print("decode_step needs a GPU", file=sys.stderr)
        return 1
    print(json.dumps(run(args.layers, args.group_size, args.trials, args.glue_pos, variants,
                         args.tp, args.stage_times)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
